"""ctypes binding of libinferd_amd.so (the C ABI declared in include/inferd_qmm.h).

The library is the only compute path: if it is missing this module raises, there is no fallback.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libinferd_amd.so")

IFD_OK, IFD_ERR_ARG, IFD_ERR_WORKSPACE, IFD_ERR_LAUNCH, IFD_ERR_UNSUPPORTED = range(5)

_vp = ctypes.c_void_p
_i = ctypes.c_int
_u32 = ctypes.c_uint32
_sz = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/inferd_qmm.h
_GEMM_ARGS = [_vp, _i, _vp, _vp, _vp, _i, _i, _i, _u32, _vp, _i, _i, _i, _vp, _sz, _vp]
SIGNATURES = {
    "ifd_version": (_i, []),
    "ifd_status_str": (ctypes.c_char_p, [_i]),
    "ifd_last_error": (ctypes.c_char_p, []),
    "ifd_workspace_check": (_i, [_vp, _sz, _vp]),
    "ifd_workspace_reset": (_i, [_vp, _sz, _vp]),
    "ifd_probe_stream_read": (_i, [_vp, _sz, _vp, _i, _vp]),
    "ifd_probe_mfma": (_i, [_i, _i, _i, _vp, _vp]),
    "ifd_gemm_w4_workspace": (_sz, [_i, _i, _i]),
    "ifd_qmv_w4": (_i, _GEMM_ARGS),
    "ifd_qmm_w4": (_i, _GEMM_ARGS),
    "ifd_gemm_w4": (_i, _GEMM_ARGS),
    "ifd_flip_w4": (_i, [_vp, _sz, _u32, _vp]),
    "ifd_silu_mul": (_i, [_vp, _vp, _i, _i, _vp]),
    "ifd_rmsnorm": (_i, [_vp, _i, _vp, _vp, _i, _i, _i, ctypes.c_float, _vp]),
    "ifd_a8_quant": (_i, [_vp, _i, _i, _i, _i, _vp, _vp, _vp]),
    "ifd_rmsnorm_a8": (_i, [_vp, _i, _vp, _vp, _i, _i, _i, ctypes.c_float, _i, _vp, _vp, _vp]),
    "ifd_silu_mul_a8": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp]),
    "ifd_splitk_res_norm": (_i, [_vp, _i, _vp, _i, _vp, _vp, _i, _i, _i, ctypes.c_float, _i, _vp, _vp, _vp]),
    "ifd_qmm_w4a8": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _i, _i, _i, _u32, _vp, _i, _i, _i, _vp, _sz, _vp]),
    "ifd_qmm_w4a8_workspace": (_sz, [_i, _i, _i]),
    "ifd_gemm_w8_workspace": (_sz, [_i, _i, _i]),
    "ifd_gemm_w8": (_i, _GEMM_ARGS),
    "ifd_qmm_w8a8": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _i, _i, _i, _u32, _vp, _i, _i, _i, _vp, _sz, _vp]),
    "ifd_qmm_w8a8_workspace": (_sz, [_i, _i, _i]),
    "ifd_t64_bytes": (_sz, [_i, _i, _i]),
    "ifd_pack_t64": (_i, [_vp, _vp, _vp, _i, _i, _i, _u32, _i, _vp, _vp]),
    "ifd_gemm_t64_workspace": (_sz, [_i, _i, _i]),
    "ifd_gemm_t64": (_i, [_vp, _i, _vp, _i, _i, _vp, _i, _i, _i, _vp, _sz, _vp]),
    "ifd_gemm_t64_noalloc": (_i, [_vp, _i, _vp, _i, _i, _vp, _i, _i, _i, _vp]),
    "ifd_gemm_t64_multi_workspace": (_sz, [_i, _i, _vp, _i]),
    "ifd_gemm_t64_multi": (_i, [_vp, _i, _i, _vp, _vp, _i, _vp, _vp, _i, _i, _vp, _sz, _vp]),
    "ifd_gemm_t64_swiglu_workspace": (_sz, [_i, _i, _i]),
    "ifd_gemm_t64_swiglu": (_i, [_vp, _i, _vp, _i, _i, _vp, _i, _i, _vp, _sz, _vp]),
    "ifd_gemm_t64_w4a8_workspace": (_sz, [_i, _i, _i]),
    "ifd_gemm_t64_w4a8": (_i, [_vp, _vp, _i, _vp, _i, _i, _vp, _i, _i, _i, _vp, _sz, _vp]),
    "ifd_t64x8_bytes": (_sz, [_i, _i]),
    "ifd_pack_t64x8": (_i, [_vp, _vp, _vp, _i, _i, _i, _u32, _vp, _vp]),
    "ifd_gemm_t64x8_workspace": (_sz, [_i, _i, _i]),
    "ifd_gemm_t64x8": (_i, [_vp, _i, _vp, _i, _i, _vp, _i, _i, _i, _vp, _sz, _vp]),
    "ifd_gemm_t64x8_w8a8_workspace": (_sz, [_i, _i, _i]),
    "ifd_gemm_t64x8_w8a8": (_i, [_vp, _vp, _i, _vp, _i, _i, _vp, _i, _i, _i, _vp, _sz, _vp]),
    "ifd_moe_router_logits": (_i, [_vp, _vp, _i, _i, _i, _i, _vp, _vp]),
    "ifd_moe_route": (_i, [_vp, _i, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp]),
    "ifd_moe_tiles_max": (_i, [_i, _i]),
    "ifd_moe_dispatch_workspace": (_sz, [_i, _i]),
    "ifd_moe_dispatch": (_i, [_vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "ifd_moe_gather": (_i, [_vp, _vp, _i, _i, _i, _vp, _vp]),
    "ifd_moe_gather_qmm": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _i, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _i, _vp]),
    "ifd_moe_gather_qmm_ex": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _i, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, _i, _vp]),
    "ifd_moe_gather_qmm_a8": (_i, [_vp, _vp, _vp, _i, _vp, _vp, _vp, _i, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _i,
                                   _vp]),
    "ifd_moe_combine": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "ifd_moe_dispatch_ex": (_i, [_vp, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "ifd_moe_t64_tile_rows": (_i, [_i, _i]),
    "ifd_moe_gather_qmm_t64_workspace": (_sz, [_i]),
    "ifd_moe_gather_qmm_t64": (_i, [_vp, _i, _vp, _i, _vp, _vp, _vp, _i, _vp, _vp, _i, _i, _i, _i, _vp, _i, _i,
                                    _vp, _sz, _vp]),
    "ifd_moe_ffn_t64_workspace": (_sz, [_i, _i, _i, _i, _i, _i]),
    "ifd_moe_ffn_t64": (_i, [_vp, _i, _i, _vp, _i, _i, _i, _i, _i, _vp, _vp, _i, _vp, _vp, _vp, _i, _vp, _vp, _vp,
                             _vp, _sz, _vp]),
    "ifd_mlp_decode_workspace": (_sz, [_i, _i, _i]),
    "ifd_mlp_decode": (_i, [_vp, _i, _vp, ctypes.c_float, _vp, _vp, _i, _i, _i, _vp, _sz, _vp]),
    "ifd_moe_decode_workspace": (_sz, [_i, _i, _i, _i, _i]),
    "ifd_moe_decode_t64_workspace": (_sz, [_i, _i, _i, _i, _i]),
    "ifd_moe_decode_t64": (_i, [_vp, _i, _i, _vp, _vp, _i, _i, _i, _i, _vp, _vp, _i, _vp, _vp, _vp, _i, _vp, _vp, _vp,
                                _vp, _vp, _sz, _vp]),
    "ifd_moe_rows_workspace": (_sz, [_i, _i, _i, _i, _i]),
    "ifd_moe_rows_t64_workspace": (_sz, [_i, _i, _i, _i, _i]),
    "ifd_moe_rows_t64": (_i, [_vp, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _i, _vp, _sz,
                              _vp]),
    "ifd_moe_rows": (_i, [_vp, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp, _vp, _i, _vp, _sz,
                          _vp]),
    "ifd_moe_decode": (_i, [_vp, _i, _i, _vp, _i, _i, _i, _i,
                            _vp, _vp, _vp, _vp, _vp, _vp, _i,
                            _vp, _vp, _vp, _vp, _vp, _vp,
                            _vp, _i, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "ifd_moe_decode_logits": (_i, [_vp, _vp, _i, _i, _i, _i, _i, _i,
                                   _vp, _vp, _vp, _vp, _vp, _vp, _i,
                                   _vp, _vp, _vp, _vp, _vp, _vp,
                                   _vp, _i, _vp, _vp, _vp, _vp, _sz, _vp]),
    "ifd_moe_decode_ex": (_i, [_vp, _i, _i, _vp, _i, _i, _i, _i,
                               _vp, _vp, _vp, _vp, _vp, _vp, _i,
                               _vp, _vp, _vp, _vp, _vp, _vp, _i,
                               _vp, _i, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "ifd_moe_decode_logits_ex": (_i, [_vp, _vp, _i, _i, _i, _i, _i, _i,
                                      _vp, _vp, _vp, _vp, _vp, _vp, _i,
                                      _vp, _vp, _vp, _vp, _vp, _vp, _i,
                                      _vp, _i, _vp, _vp, _vp, _vp, _sz, _vp]),
    "ifd_moe_ffn_workspace": (_sz, [_i, _i, _i, _i, _i, _i]),
    "ifd_moe_ffn": (_i, [_vp, _i, _i, _vp, _i, _i, _i, _i, _i,
                         _vp, _vp, _vp, _vp, _vp, _vp, _i,
                         _vp, _vp, _vp, _vp, _vp, _vp, _i,
                         _vp, _i, _vp, _vp, _vp, _vp, _sz, _vp]),
}

_lib = None


class IfdError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"inferd_amd status {status}: {msg}")
        self.status = status


def lib():
    """Load libinferd_amd.so (raises if it has not been built: no fallback path exists)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run `python -m inferd_amd.build` (HIP extension required)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(status: int) -> None:
    if status != IFD_OK:
        raise IfdError(status, (lib().ifd_last_error() or b"").decode())
