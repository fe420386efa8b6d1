"""CPU checks of the C ABI boundary: the library loads, exports every symbol include/inferd_qmm.h declares, and
rejects invalid requests with status codes before touching the GPU (no compute runs here)."""
import ctypes
import os
import re

import pytest

from inferd_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "inferd_qmm.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ifd_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    syms = declared_symbols()
    for s in ["ifd_gemm_w4", "ifd_qmv_w4", "ifd_qmm_w4", "ifd_a8_quant", "ifd_qmm_w4a8", "ifd_moe_route",
              "ifd_moe_dispatch", "ifd_moe_gather_qmm", "ifd_moe_combine", "ifd_moe_ffn"]:
        assert s in syms


def test_library_exports_every_declared_symbol():
    L = ctypes.CDLL(_lib.LIB_PATH)
    missing = [s for s in declared_symbols() if not hasattr(L, s)]
    assert not missing, missing
    # and the Python binding covers the same set
    assert set(declared_symbols()) == set(_lib.SIGNATURES)


def test_status_strings_and_version():
    L = _lib.lib()
    assert L.ifd_version() == 1
    assert L.ifd_status_str(0) == b"ok"
    assert L.ifd_status_str(2) == b"workspace too small"


@pytest.mark.parametrize("kw,msg", [
    (dict(K=100), b"multiple of the group size"),
    (dict(mode=3), b"mode=3"),
    (dict(xr=0x1234), b"xr="),
    (dict(lda=64), b"lda="),
    (dict(ldk=96), b"ldk="),
    (dict(wq=None), b"null pointer"),
    (dict(wq=8), b"16-byte aligned"),
])
def test_gemm_rejects_bad_arguments(kw, msg):
    L = _lib.lib()
    a = dict(A=4096, lda=128, wq=4096, s=4096, b=4096, N=64, K=128, ldk=0, xr=0, C=4096, ldc=64, M=4, mode=0)
    a.update(kw)
    if "K" in kw and "lda" not in kw:
        a["lda"] = max(a["lda"], kw["K"] + (-kw["K"]) % 8)
    for fn in (L.ifd_gemm_w4, L.ifd_qmv_w4, L.ifd_qmm_w4):
        rc = fn(a["A"], a["lda"], a["wq"], a["s"], a["b"], a["N"], a["K"], a["ldk"], a["xr"], a["C"], a["ldc"], a["M"],
                a["mode"], None, 0, None)
        assert rc == _lib.IFD_ERR_ARG
        assert msg in L.ifd_last_error()


def test_qmv_rejects_large_m_and_moe_rejects_bad_shapes():
    L = _lib.lib()
    rc = L.ifd_qmv_w4(4096, 128, 4096, 4096, 4096, 64, 128, 0, 0, 4096, 64, 129, 0, None, 0, None)
    assert rc == _lib.IFD_ERR_ARG and b"M <= 128" in L.ifd_last_error()
    assert L.ifd_moe_route(4096, 0, 4, 600, 10, 601, 1, 1, 4096, 4096, 4096, None) == _lib.IFD_ERR_ARG
    assert L.ifd_moe_route(4096, 0, 4, 512, 17, 513, 1, 1, 4096, 4096, 4096, None) == _lib.IFD_ERR_ARG
    assert L.ifd_moe_route(4096, 0, 4, 512, 10, 512, 1, 1, 4096, 4096, 4096, None) == _lib.IFD_ERR_ARG
    assert L.ifd_moe_dispatch(4096, 10, 2000, 4096, 4096, 4096, 4096, 4096, None, 0, None) == _lib.IFD_ERR_ARG


HEADER_BYTES = 4096  # the counters every workspace starts with


def test_workspace_queries():
    L = _lib.lib()
    # decode shapes split K: the counter header + partials S * M * N fp32
    ws = L.ifd_gemm_w4_workspace(1, 5120, 5120)
    assert ws > HEADER_BYTES and (ws - HEADER_BYTES) % (5120 * 4) == 0
    assert L.ifd_gemm_w4_workspace(4096, 17408, 5120) == 0
    ws = L.ifd_gemm_t64_workspace(1, 34816, 5120)
    assert ws > HEADER_BYTES and (ws - HEADER_BYTES) % (34816 * 4) == 0
    # the SwiGLU entry needs the bf16 product in the workspace even without a split
    assert L.ifd_gemm_t64_workspace(4, 1024, 256) == 0
    assert L.ifd_gemm_t64_swiglu_workspace(4, 1024, 256) == HEADER_BYTES + 4 * 1024 * 2
    assert L.ifd_moe_ffn_workspace(2048, 2048, 512, 512, 10, 512) > 2048 * 10 * 2048 * 2
    assert L.ifd_moe_tiles_max(20480, 512) == 640 + 512
    # a too-small workspace is refused before any launch
    rc = L.ifd_qmv_w4(4096, 5120, 4096, 4096, 4096, 5120, 5120, 0, 0, 4096, 5120, 1, 0, None, 0, None)
    assert rc == _lib.IFD_ERR_WORKSPACE
    rc = L.ifd_gemm_t64(4096, 5120, 4096, 34816, 5120, 4096, 34816, 1, 0, 4096, HEADER_BYTES, None)
    assert rc == _lib.IFD_ERR_WORKSPACE


def test_t64_w4a8_argument_checks():
    """Per-group activations (per_token = 0) need the workspace the size query reports (its int8-to-bf16 staging and
    transposed scales); any per_token other than 0 or 1 is refused. Both before any GPU work."""
    L = _lib.lib()
    rc = L.ifd_gemm_t64_w4a8(4096, 4096, 0, 4096, 256, 256, 4096, 256, 4, 0, None, 0, None)
    assert rc == _lib.IFD_ERR_WORKSPACE and b"workspace" in L.ifd_last_error()
    assert L.ifd_gemm_t64_w4a8_workspace(4, 256, 256) > 4096 + 4 * 256 * 2
    rc = L.ifd_gemm_t64_w4a8(4096, 4096, 3, 4096, 256, 256, 4096, 256, 4, 0, None, 0, None)
    assert rc == _lib.IFD_ERR_ARG and b"per_token=3" in L.ifd_last_error()


def test_moe_decode_ex_refuses_other_shared_widths():
    """The decode MoE takes a 4- or 8-bit shared expert (moe_gu2_4_4 / moe_gu2_4_8), the gathered GEMM 4- or 8-bit
    stacks; any other width is refused before any GPU work."""
    L = _lib.lib()
    args = [4096, 4, 2048, 4096, 512, 10, 1, 1, 4096, 4096, 4096, 4096, 4096, 4096, 512,
            4096, 4096, 4096, 4096, 4096, 4096, 6, 4096, 0, None, None, None, None, None, 0, None]
    assert L.ifd_moe_decode_ex(*args) == _lib.IFD_ERR_ARG and b"shared_bits=6" in L.ifd_last_error()
    la = [4096, 4096, 4, 2048, 512, 10, 1, 1, 4096, 4096, 4096, 4096, 4096, 4096, 512,
          4096, 4096, 4096, 4096, 4096, 4096, 3, 4096, 0, None, None, None, None, 0, None]
    assert L.ifd_moe_decode_logits_ex(*la) == _lib.IFD_ERR_ARG and b"shared_bits=3" in L.ifd_last_error()
    # the gathered expert GEMM: 4- or 8-bit stacks
    assert L.ifd_moe_gather_qmm_ex(4096, None, 1, 4096, 4096, 4096, 4, 4096, 4096, 4096, 8, 256, 256, 2, 0, 4096, 32,
                                   None) == _lib.IFD_ERR_ARG and b"bits=2" in L.ifd_last_error()


def test_t64x8_refuses_bad_arguments():
    """The 8-bit T64x8 entry points: per-group activation scales, K % 64, the 4-bit flip mask and its size query."""
    L = _lib.lib()
    rc = L.ifd_gemm_t64x8_w8a8(4096, 4096, 0, 4096, 256, 256, 4096, 256, 4, 0, None, 0, None)
    assert rc == _lib.IFD_ERR_UNSUPPORTED and b"per-token" in L.ifd_last_error()
    assert L.ifd_gemm_t64x8_w8a8(4096, 4096, 1, 4096, 256, 96, 4096, 256, 4, 0, None, 0, None) == _lib.IFD_ERR_ARG
    assert L.ifd_pack_t64x8(4096, 4096, 4096, 64, 128, 0, 0x88888888, 4096, None) == _lib.IFD_ERR_ARG
    assert b"0x80808080" in L.ifd_last_error()
    assert L.ifd_t64x8_bytes(64, 96) == 0 and L.ifd_t64x8_bytes(200, 128) == 2 * 7 * 2176
    assert L.ifd_gemm_t64x8_w8a8_workspace(2048, 5120, 5120) > HEADER_BYTES


def test_new_entry_points_reject_bad_arguments():
    """8-bit GEMM / W8A8, the decode MoE, the MLP block and the int8 gathered GEMM return IFD_ERR_ARG with a reason
    before any GPU work."""
    L = _lib.lib()
    E = _lib.IFD_ERR_ARG
    # 8-bit weights: the 4-bit flip mask is not an 8-bit one
    assert L.ifd_gemm_w8(4096, 128, 4096, 4096, 4096, 64, 128, 0, 0x88888888, 4096, 64, 4, 0, None, 0, None) == E
    assert b"0x80808080" in L.ifd_last_error()
    assert L.ifd_qmm_w8a8(4096, 4096, 0, 4096, 4096, 4096, 64, 100, 0, 0, 4096, 64, 4, 0, None, 0, None) == E
    # quantizer forms 0, 1, 2 only
    assert L.ifd_a8_quant(4096, 128, 4, 128, 3, 4096, 4096, None) == E and b"per_token=3" in L.ifd_last_error()
    # 16-byte activation loads and 8-byte code stores: aligned A, lda % 8 == 0, aligned U
    assert L.ifd_a8_quant(4098, 128, 4, 128, 0, 4096, 4096, None) == E and b"aligned" in L.ifd_last_error()
    assert L.ifd_a8_quant(4096, 132, 4, 128, 0, 4096, 4096, None) == E and b"lda=132" in L.ifd_last_error()
    assert L.ifd_a8_quant(4096, 128, 4, 128, 0, 4100, 4096, None) == E and b"aligned" in L.ifd_last_error()
    # decode MoE: at most 16 tokens, H a multiple of 512, k <= 16, no shared gate without a shared expert
    args = [4096, 17, 2048, 4096, 512, 10, 1, 0, 4096, 4096, 4096, 4096, 4096, 4096, 512,
            None, None, None, None, None, None, 4096, 0, None, None, None, None, None, 0, None]
    assert L.ifd_moe_decode(*args) == E and b"T <= 16" in L.ifd_last_error()
    # the same checks from caller logits
    assert L.ifd_moe_decode_logits(4096, 4096, 17, 2048, 512, 10, 1, 0, 4096, 4096, 4096, 4096, 4096, 4096, 512,
                                   None, None, None, None, None, None, 4096, 0, None, None, None, None, 0,
                                   None) == E and b"T <= 16" in L.ifd_last_error()
    a = list(args); a[1], a[2] = 4, 1280
    assert L.ifd_moe_decode(*a) == E and b"H multiple of 512" in L.ifd_last_error()
    a = list(args); a[1], a[5] = 4, 17
    assert L.ifd_moe_decode(*a) == E
    a = list(args); a[1], a[7] = 4, 1
    assert L.ifd_moe_decode(*a) == E and b"shared gate" in L.ifd_last_error()
    # the MLP block: H and I multiples of 256
    assert L.ifd_mlp_decode(4096, 5120, 4096, 1e-6, 4096, 4096, 4, 5120, 1000, None, 0, None) == E
    # int8 gathered GEMM: K a multiple of 64, an even N for silu
    assert L.ifd_moe_gather_qmm_a8(4096, 4096, None, 1, 4096, 4096, 4096, 4, 4096, 4096, 4096, 8, 64, 100, 0, 4096, 32,
                                   None) == E
    assert L.ifd_moe_gather_qmm_a8(4096, 4096, None, 1, 4096, 4096, 4096, 4, 4096, 4096, 4096, 8, 63, 128, 1, 4096, 32,
                                   None) == E


def test_new_workspace_queries():
    L = _lib.lib()
    assert L.ifd_moe_decode_workspace(17, 2048, 512, 512, 10) == 0 and L.ifd_moe_decode_workspace(16, 2048, 512, 512, 10) > 0
    w1, w8 = L.ifd_moe_decode_workspace(1, 2048, 512, 512, 10), L.ifd_moe_decode_workspace(8, 2048, 512, 512, 10)
    assert HEADER_BYTES < w1 < w8
    assert L.ifd_mlp_decode_workspace(1, 5120, 17408) > HEADER_BYTES + 5120 * 2 + 17408 * 2
    assert L.ifd_gemm_w8_workspace(1, 5120, 5120) == L.ifd_gemm_w4_workspace(1, 5120, 5120)


def test_multi_linear_gemv_checks():
    """The multi-linear decode GEMV: 1 to 8 linears, M <= 16, K a multiple of 256, ldc >= N per linear, and a K split
    needs the workspace (with its counter header) the size query reports. All before any GPU work."""
    L = _lib.lib()
    E = _lib.IFD_ERR_ARG

    def arrs(Ns, ldcs=None):
        n = len(Ns)
        return ((ctypes.c_void_p * n)(*[4096] * n), (ctypes.c_int * n)(*Ns), (ctypes.c_void_p * n)(*[4096] * n),
                (ctypes.c_int * n)(*(ldcs or Ns)))

    Ns = [5120, 1024, 1024, 5120]
    wts, ns, cs, ldcs = arrs(Ns)
    need = L.ifd_gemm_t64_multi_workspace(1, 4, ns, 5120)
    assert need > HEADER_BYTES and (need - HEADER_BYTES) % (4 * 32 * 4) == 0
    assert L.ifd_gemm_t64_multi_workspace(17, 4, ns, 5120) == 0
    assert L.ifd_gemm_t64_multi_workspace(1, 9, (ctypes.c_int * 9)(*[128] * 9), 5120) == 0
    assert L.ifd_gemm_t64_multi_workspace(1, 4, ns, 5000) == 0
    call = lambda n=4, M=1, K=5120, mode=0, a=(wts, ns, cs, ldcs), ws=4096, wsb=0: L.ifd_gemm_t64_multi(
        4096, K, n, a[0], a[1], K, a[2], a[3], M, mode, ws, wsb, None)
    assert call(n=0) == E and call(n=9) == E and b"1 to 8" in L.ifd_last_error()
    assert call(M=17) == E and call(K=5000) == E
    assert call(mode=3) == E and b"mode=3" in L.ifd_last_error()
    assert call(a=arrs(Ns, [5120, 1000, 1024, 5120])) == E and b"linear 1" in L.ifd_last_error()
    assert call() == _lib.IFD_ERR_WORKSPACE
    assert call(ws=None, wsb=need) == _lib.IFD_ERR_WORKSPACE
    assert call(M=0) == _lib.IFD_OK


def test_moe_rows_checks():
    """The per-row MoE on the caller's routing: the decode kernels' shapes (H multiple of 512, I of 64, E <= 512,
    k <= 16), the routing arrays, and the shared rows' gate weights; any T, with one workspace size from 16 tokens
    up. All before any GPU work."""
    L = _lib.lib()
    E = _lib.IFD_ERR_ARG
    assert L.ifd_moe_rows_workspace(16, 2048, 512, 512, 10) == L.ifd_moe_decode_workspace(16, 2048, 512, 512, 10) > 0
    assert L.ifd_moe_rows_workspace(300, 2048, 512, 512, 10) == L.ifd_moe_rows_workspace(16, 2048, 512, 512, 10)
    call = lambda T=20, H=2048, Ex=512, k=10, idx=4096, sg=4096, I=512, ys=4096: L.ifd_moe_rows(
        4096, T, H, Ex, k, idx, 4096, sg, 4096, 4096, 4096, 4096, 4096, 4096, I, ys, 4096, 0, 4096, 0, None)
    assert call(H=1280) == E and b"H multiple of 512" in L.ifd_last_error()
    assert call(Ex=513) == E and call(k=17) == E and call(I=100) == E
    assert call(idx=None) == E and b"null" in L.ifd_last_error()
    assert call(sg=None) == E and b"gate weights" in L.ifd_last_error()
    assert call(T=0) == _lib.IFD_OK
    assert call() == _lib.IFD_ERR_WORKSPACE  # no workspace past the header
    # on T64 stacks: 16-token launch groups, one workspace size from 16 tokens up, the same checks
    assert L.ifd_moe_rows_t64_workspace(300, 2048, 512, 512, 10) == L.ifd_moe_rows_t64_workspace(16, 2048, 512, 512, 10)
    assert L.ifd_moe_rows_t64_workspace(16, 2048, 512, 512, 10) >= L.ifd_moe_decode_t64_workspace(16, 2048, 512, 512,
                                                                                                  10)
    assert L.ifd_moe_decode_t64_workspace(17, 2048, 512, 512, 10) == 0
    call64 = lambda T=20, H=2048, Ex=512, k=10, idx=4096, sg=4096, I=512, ys=4096, sw=None: L.ifd_moe_rows_t64(
        4096, T, H, Ex, k, idx, 4096, sg, 4096, 4096, I, sw, sw, ys, 4096, 0, 4096, 0, None)
    assert call64(H=1280) == E and b"H multiple of 512" in L.ifd_last_error()
    assert call64(Ex=513) == E and call64(k=17) == E and call64(I=100) == E
    assert call64(idx=None) == E and b"null" in L.ifd_last_error()
    assert call64(sg=None) == E and b"gate weights" in L.ifd_last_error()
    assert call64(sw=4096) == E and b"not both" in L.ifd_last_error()
    assert call64(sw=4096, ys=None, sg=None) == E and b"gate weights" in L.ifd_last_error()
    assert call64(T=0) == _lib.IFD_OK
    assert call64() == _lib.IFD_ERR_WORKSPACE
    assert call64(sw=4096, ys=None) == _lib.IFD_ERR_WORKSPACE
