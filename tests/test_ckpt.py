"""The checkpoint loader (inferd_amd/csrc/ckpt.h; reference engine/src/weights.h:54-406, moe.h:14-87, qwen4.h:11-29)
through its host-only test program, tests/cpp/ckpt_test.cpp, on MLX-style safetensors files written here by the
`safetensors` package, and the oracle's load-time quantizer against hand-derived answers. CPU only."""
import json
import os
import struct
import subprocess
from fractions import Fraction

import numpy as np
import pytest

from oracle import oracle as orc

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "ckpt_test")


def _need_bin():
    if not os.path.exists(BIN):
        pytest.skip("tests/cpp/ckpt_test is not built (python tests/cpp/build.py)")


def _save(path, tensors, metadata=None):
    """tensors: name -> numpy uint32 (U32) or ('bf16', uint16 bit patterns) (BF16)."""
    import torch
    from safetensors.torch import save_file
    t = {}
    for k, v in tensors.items():
        if isinstance(v, tuple):
            t[k] = torch.from_numpy(np.array(v[1], np.uint16)).view(torch.bfloat16)
        else:
            t[k] = torch.from_numpy(np.array(v))  # copies: safetensors refuses tensors that share memory
    save_file(t, path, metadata=metadata or {"format": "mlx"})


def _run(cmd, src, out, *args):
    _need_bin()
    return subprocess.run([BIN, cmd, str(src), str(out), *map(str, args)], capture_output=True, text=True, timeout=60)


def _load(cmd, src, tmp_path, *args):
    out = tmp_path / "out.bin"
    r = _run(cmd, src, out, *args)
    assert r.returncode == 0, r.stderr
    raw = out.read_bytes()
    bits, E, N, K = struct.unpack("<4i", raw[:16])
    o = 16
    res = {"bits": bits, "E": E, "N": N, "K": K}
    if bits == 16:
        res["w16"] = np.frombuffer(raw, np.uint16, N * K, o)
        return res
    nw = E * N * K * bits // 32
    ns = E * N * (K // 64)
    res["wq"] = np.frombuffer(raw, np.uint32, nw, o)
    o += nw * 4
    res["s"] = np.frombuffer(raw, np.uint16, ns, o)
    o += ns * 2
    res["b"] = np.frombuffer(raw, np.uint16, ns, o)
    assert o + ns * 2 == len(raw)
    return res


def _qpart(rng, n, K, bits=4, gs=64, lead=()):
    """An MLX-quantized part: U32 weight [*lead, n, K bits/32], bf16 scales / biases [*lead, n, K / gs]."""
    wq = rng.integers(0, 2 ** 32, size=(*lead, n, K * bits // 32), dtype=np.uint32)
    s = orc.f32_to_bf16(rng.uniform(0.001, 0.02, size=(*lead, n, K // gs)).astype(np.float32))
    b = orc.f32_to_bf16(rng.uniform(-0.1, 0.1, size=(*lead, n, K // gs)).astype(np.float32))
    return wq, s, b


def _put(d, prefix, part):
    d[prefix + ".weight"] = part[0]
    d[prefix + ".scales"] = ("bf16", part[1])
    d[prefix + ".biases"] = ("bf16", part[2])


# ---- the oracle's quantizer, pinned by hand-derived answers ---------------------------------------------------------
def test_quantize_affine_known_answer_ramp():
    """Values 0..63, 4 bits: lo = 0, sc = 63 / 15 = 4.2 -> bf16 4.1875 = 67/16, so q_i = floor(16 i / 67 + 1/2) in
    exact arithmetic (no tie can occur: 67 is odd)."""
    w = orc.f32_to_bf16(np.arange(64, dtype=np.float32)[None])
    wq, s, b, codes = orc.quantize_affine(w, 4)
    assert orc.bf16_to_f32(s)[0, 0] == 4.1875 and orc.bf16_to_f32(b)[0, 0] == 0.0
    want = [int(Fraction(16 * i, 67) + Fraction(1, 2)) for i in range(64)]
    assert codes[0].tolist() == want
    assert codes[0, 63] == 15 and codes[0, 0] == 0
    # packing: element j of word at bits 4 j, low first
    assert int(wq[0, 0]) == sum(want[j] << (4 * j) for j in range(8))


def test_quantize_affine_ties_round_away_and_special_groups():
    """Group 0: lo = -1, hi = 14, sc = 1 exactly: w = 1.5 -> v = 2.5 rounds away from zero to 3 (half-even would give
    2), w = 0.5 -> 2 (1.5 away). Group 1: constant -> sc = 1e-8, every code 0, bias = the value. Group 2: all
    negative, 8 bits: -3 .. -3 + 255 / 128 on a 1/128 grid, sc = 1/128 exactly, q = 128 (w + 3)."""
    g0 = np.zeros(64, np.float32)
    g0[0], g0[1], g0[2], g0[3] = -1, 14, 1.5, 0.5
    g1 = np.full(64, -0.375, np.float32)
    w4 = orc.f32_to_bf16(np.concatenate([g0, g1])[None])
    _, s, b, c = orc.quantize_affine(w4, 4)
    sf, bf = orc.bf16_to_f32(s)[0], orc.bf16_to_f32(b)[0]
    assert sf[0] == 1.0 and bf[0] == -1.0
    assert c[0, :4].tolist() == [0, 15, 3, 2] and (c[0, 4:64] == 1).all()
    assert bf[1] == -0.375 and sf[1] == orc.bf16_to_f32(orc.f32_to_bf16(np.float32(1e-8)))
    assert (c[0, 64:] == 0).all()
    steps = np.arange(64) * 4 % 256
    steps[0], steps[1] = 0, 255
    g2 = (-3 + steps / 128).astype(np.float32)
    _, s8, b8, c8 = orc.quantize_affine(orc.f32_to_bf16(g2[None]), 8)
    assert orc.bf16_to_f32(s8)[0, 0] == 1 / 128 and orc.bf16_to_f32(b8)[0, 0] == -3
    assert c8[0].tolist() == steps.tolist()


def test_quantize_affine_error_bound():
    """Every dequantized value is within half a step of its input, except where the clamp cuts: rounding the scale to
    bf16 (relative error up to 2^-8) can shrink it so that the group maximum maps to levels (1 + 2^-8), up to about
    one step above the top code at 8 bits. The group minimum gets code 0; the maximum gets the top code at 4 bits
    (15 / (1 + 2^-8) still rounds to 15) and at least one below it at 8 bits (255 / (1 + 2^-8) may round to 254)."""
    rng = np.random.default_rng(5)
    w = orc.f32_to_bf16(rng.standard_normal((8, 512)).astype(np.float32))
    for bits in (4, 8):
        wq, s, b, codes = orc.quantize_affine(w, bits)
        sf = orc.bf16_to_f32(s).astype(np.float64).repeat(64, axis=1)
        bf = orc.bf16_to_f32(b).astype(np.float64).repeat(64, axis=1)
        x = orc.bf16_to_f32(w).astype(np.float64)
        err = np.abs(sf * codes + bf - x)
        bound = max(0.5, ((1 << bits) - 1) * 2 ** -8 * 1.01)
        assert (err <= sf * bound).all(), (bits, (err / sf).max())
        if bits == 4:
            assert (err / sf).max() <= 0.5
        g = x.reshape(8, 8, 64)
        cg = codes.reshape(8, 8, 64)
        assert (np.take_along_axis(cg, g.argmin(-1)[..., None], -1) == 0).all()
        top = np.take_along_axis(cg, g.argmax(-1)[..., None], -1)
        assert (top == 15).all() if bits == 4 else (top >= 254).all()
        assert (orc.pack_affine(codes, bits) == wq).all()


# ---- the loader ---------------------------------------------------------------------------------------------------
def test_qlinear_fused_rows_across_shards(tmp_path):
    """gate and up in two shard files, fused by rows in the order named (reference load_qlinear, weights.h:271-340)."""
    rng = np.random.default_rng(1)
    K = 512
    gate, up = _qpart(rng, 96, K), _qpart(rng, 160, K)
    d0, d1 = {}, {}
    _put(d0, "mlp.gate_proj", gate)
    _put(d1, "mlp.up_proj", up)
    _save(tmp_path / "model-00001-of-00002.safetensors", d0)
    _save(tmp_path / "model-00002-of-00002.safetensors", d1)
    r = _load("qlinear", tmp_path, tmp_path, "mlp.gate_proj", "mlp.up_proj")
    assert (r["bits"], r["N"], r["K"]) == (4, 256, K)
    assert (r["wq"].reshape(256, -1) == np.concatenate([gate[0], up[0]])).all()
    assert (r["s"].reshape(256, -1) == np.concatenate([gate[1], up[1]])).all()
    assert (r["b"].reshape(256, -1) == np.concatenate([gate[2], up[2]])).all()
    r2 = _load("qlinear", tmp_path, tmp_path, "mlp.up_proj", "mlp.gate_proj")
    assert (r2["wq"].reshape(256, -1)[:160] == up[0]).all()


def test_qlinear_8bit_and_group_expansion_from_config(tmp_path):
    """config.json quantization {bits 4, group_size 128} with an 8-bit group-64 override for one prefix: the 4-bit
    group-128 part is expanded to 64-groups (scale and bias repeated), the override loads as 8-bit
    (reference qspec, qwen4.h:11-29; the expansion of load_moe, moe.h:69-83)."""
    rng = np.random.default_rng(2)
    K = 1024
    p4 = _qpart(rng, 64, K, bits=4, gs=128)
    p8 = _qpart(rng, 32, K, bits=8, gs=64)
    d = {}
    _put(d, "a", p4)
    _put(d, "lm_head", p8)
    _save(tmp_path / "model.safetensors", d)
    (tmp_path / "config.json").write_text(json.dumps(
        {"model_type": "x", "quantization": {"bits": 4, "group_size": 128, "lm_head": {"bits": 8, "group_size": 64}}}))
    r = _load("qlinear", tmp_path, tmp_path, "a")
    assert (r["bits"], r["N"], r["K"]) == (4, 64, K)
    assert (r["wq"].reshape(64, -1) == p4[0]).all()
    assert (r["s"].reshape(64, -1) == orc.expand_groups(p4[1], 128)).all()
    assert (r["b"].reshape(64, -1) == orc.expand_groups(p4[2], 128)).all()
    r8 = _load("qlinear", tmp_path, tmp_path, "lm_head")
    assert (r8["bits"], r8["N"], r8["K"]) == (8, 32, K)
    assert (r8["wq"].reshape(32, -1) == p8[0]).all() and (r8["s"].reshape(32, -1) == p8[1]).all()


def test_qlinear_group128_expansion_dequantizes_identically(tmp_path):
    """The expansion is exact: dequantizing the loaded 64-group layout gives, element for element, the group-128
    dequantization s[k // 128] q + b[k // 128] of the file."""
    rng = np.random.default_rng(3)
    K = 256
    p = _qpart(rng, 16, K, bits=4, gs=128)
    d = {}
    _put(d, "w", p)
    _save(tmp_path / "model.safetensors", d)
    (tmp_path / "config.json").write_text(json.dumps({"quantization": {"bits": 4, "group_size": 128}}))
    r = _load("qlinear", tmp_path, tmp_path, "w")
    got = orc.dequant_f32(r["wq"].reshape(16, -1), r["s"].reshape(16, -1), r["b"].reshape(16, -1), K)
    codes = orc.unpack_w4(p[0], K).astype(np.float32)
    sf = orc.bf16_to_f32(p[1]).repeat(128, axis=1)
    bf = orc.bf16_to_f32(p[2]).repeat(128, axis=1)
    assert (got == (sf * codes + bf).astype(np.float32)).all()


def test_qlinear_bf16_passthrough_and_load_time_quantization(tmp_path):
    """BF16 weights load unchanged as bits 16 (weights.h:273-296); load_qlinear_bf16 quantizes the fused rows at load
    bit-exactly as the oracle's restatement of load_qlinear_bf16_q8 (weights.h:349-406), and quantize_affine on raw
    rows agrees."""
    rng = np.random.default_rng(4)
    K = 384
    a = orc.f32_to_bf16(rng.standard_normal((40, K)).astype(np.float32))
    b = orc.f32_to_bf16((rng.standard_normal((24, K)) * 3).astype(np.float32))
    a[0, :64] = a[0, 0]  # a constant group
    _save(tmp_path / "model.safetensors", {"x.weight": ("bf16", a), "y.weight": ("bf16", b)})
    r = _load("qlinear", tmp_path, tmp_path, "x", "y")
    assert (r["bits"], r["N"], r["K"]) == (16, 64, K)
    assert (r["w16"].reshape(64, K) == np.concatenate([a, b])).all()
    both = np.concatenate([a, b])
    for bits in (4, 8):
        wq, s, bb, _ = orc.quantize_affine(both, bits)
        q = _load("bf16q", tmp_path, tmp_path, bits, "x.weight", "y.weight")
        assert (q["bits"], q["N"], q["K"]) == (bits, 64, K)
        assert (q["wq"] == wq.reshape(-1)).all() and (q["s"] == s.reshape(-1)).all() and (q["b"] == bb.reshape(-1)).all()
        raw = tmp_path / "raw.bin"
        raw.write_bytes(both.tobytes())
        q2 = _load("quant", raw, tmp_path, bits, 64, K)
        assert (q2["wq"] == wq.reshape(-1)).all() and (q2["s"] == s.reshape(-1)).all()


def test_moe_stacks_fused_per_expert_with_group_expansion(tmp_path):
    """switch_mlp gate / up stacks [E, n, .] fused along N per expert, group 128 expanded (reference load_moe,
    moe.h:14-87); a 2-D part loads as E = 1."""
    rng = np.random.default_rng(6)
    E, I, H = 4, 64, 256
    g, u = _qpart(rng, I, H, gs=128, lead=(E,)), _qpart(rng, I, H, gs=128, lead=(E,))
    d = {}
    _put(d, "mlp.switch_mlp.gate_proj", g)
    _put(d, "mlp.switch_mlp.up_proj", u)
    sh = _qpart(rng, 32, H, gs=128)
    _put(d, "mlp.shared_expert.gate_proj", sh)
    _save(tmp_path / "model.safetensors", d)
    (tmp_path / "config.json").write_text(json.dumps({"quantization": {"bits": 4, "group_size": 128}}))
    r = _load("moe", tmp_path, tmp_path, "mlp.switch_mlp.gate_proj", "mlp.switch_mlp.up_proj")
    assert (r["bits"], r["E"], r["N"], r["K"]) == (4, E, 2 * I, H)
    assert (r["wq"].reshape(E, 2 * I, -1) == np.concatenate([g[0], u[0]], axis=1)).all()
    want_s = np.concatenate([orc.expand_groups(g[1], 128), orc.expand_groups(u[1], 128)], axis=1)
    want_b = np.concatenate([orc.expand_groups(g[2], 128), orc.expand_groups(u[2], 128)], axis=1)
    assert (r["s"].reshape(E, 2 * I, -1) == want_s).all() and (r["b"].reshape(E, 2 * I, -1) == want_b).all()
    r1 = _load("moe", tmp_path, tmp_path, "mlp.shared_expert.gate_proj")
    assert (r1["E"], r1["N"]) == (1, 32)
    assert (r1["s"].reshape(32, -1) == orc.expand_groups(sh[1], 128)).all()


# ---- malformed input: each is refused with a message, before anything is sized from it ------------------------------
def _raw_file(path, header: dict, data: bytes, hlen=None):
    h = json.dumps(header).encode()
    path.write_bytes(struct.pack("<Q", len(h) if hlen is None else hlen) + h + data)


@pytest.mark.parametrize("case,msg", [
    ("hlen_past_end", "header length"),
    ("offsets_outside", "outside the"),
    ("shape_vs_bytes", "shape holds"),
    ("not_json", "header"),
    ("bad_dtype", "unsupported dtype"),
    ("reversed_offsets", "outside the"),
    ("negative_dim", "expected an integer"),
])
def test_rejects_malformed_headers(tmp_path, case, msg):
    """A header is validated against the file (reference Checkpoint, weights.h:54-224): its length, each tensor's
    data_offsets against the data section and its dtype / shape against the byte range."""
    f = tmp_path / "model.safetensors"
    data = bytes(64)
    good = {"w.weight": {"dtype": "U32", "shape": [2, 8], "data_offsets": [0, 64]}}
    if case == "hlen_past_end":
        _raw_file(f, good, data, hlen=10 ** 6)
    elif case == "offsets_outside":
        _raw_file(f, {"w.weight": {"dtype": "U32", "shape": [2, 8], "data_offsets": [32, 96]}}, data)
    elif case == "shape_vs_bytes":
        _raw_file(f, {"w.weight": {"dtype": "U32", "shape": [4, 8], "data_offsets": [0, 64]}}, data)
    elif case == "not_json":
        f.write_bytes(struct.pack("<Q", 5) + b"{abc}" + data)
    elif case == "bad_dtype":
        _raw_file(f, {"w.weight": {"dtype": "Q4", "shape": [2, 8], "data_offsets": [0, 64]}}, data)
    elif case == "reversed_offsets":
        _raw_file(f, {"w.weight": {"dtype": "U8", "shape": [0], "data_offsets": [64, 0]}}, data)
    elif case == "negative_dim":
        _raw_file(f, {"w.weight": {"dtype": "U32", "shape": [-2, -8], "data_offsets": [0, 64]}}, data)
    r = _run("qlinear", tmp_path, tmp_path / "o.bin", "w")
    assert r.returncode == 2 and "ckpt error" in r.stderr and msg in r.stderr, r.stderr


def test_rejects_inconsistent_tensors(tmp_path):
    """dtype, shape, width, fusion and config errors name the tensor (reference load_qlinear / load_moe / qspec)."""
    rng = np.random.default_rng(7)
    K = 256
    d = {}
    _put(d, "ok", _qpart(rng, 8, K))
    _put(d, "k512", _qpart(rng, 8, 512))
    wq, s, b = _qpart(rng, 8, K)
    d["f32s.weight"], d["f32s.scales"], d["f32s.biases"] = wq, s.view(np.uint16).astype(np.float32), ("bf16", b)
    d["rows.weight"], d["rows.scales"], d["rows.biases"] = wq, ("bf16", s[:4]), ("bf16", b[:4])
    d["w3.weight"], d["w3.scales"], d["w3.biases"] = wq[:, :24], ("bf16", s), ("bf16", b)  # 3-bit
    _save(tmp_path / "model.safetensors", d)
    cases = [(("ok", "missing"), "missing tensor missing.weight"),
             (("f32s",), "expected BF16, got F32"),
             (("rows",), "do not match"),
             (("w3",), "not a 4- or 8-bit"),
             (("ok", "k512"), "differ in K")]
    for names, msg in cases:
        r = _run("qlinear", tmp_path, tmp_path / "o.bin", *names)
        assert r.returncode == 2 and msg in r.stderr, (names, r.stderr)
    r = _run("bf16q", tmp_path, tmp_path / "o.bin", 3, "ok.weight")
    assert r.returncode == 2 and "3-bit quantization is not supported" in r.stderr
    for cfg, msg in [({"quantization": {"bits": 4, "group_size": 96}}, "not a multiple of 64"),
                     ({"quantization": {"bits": 9}}, "quantization config"),
                     ({"quantization": {"ok": {"bits": 4}}}, "override needs bits and group_size")]:
        (tmp_path / "config.json").write_text(json.dumps(cfg))
        r = _run("qlinear", tmp_path, tmp_path / "o.bin", "ok")
        assert r.returncode == 2 and msg in r.stderr, (cfg, r.stderr)
    (tmp_path / "config.json").write_text("{not json")
    r = _run("qlinear", tmp_path, tmp_path / "o.bin", "ok")
    assert r.returncode == 2 and "JSON" in r.stderr


def test_truncated_file_is_refused(tmp_path):
    """A file cut short after a valid header: its tensors fall outside the data section."""
    rng = np.random.default_rng(8)
    d = {}
    _put(d, "w", _qpart(rng, 8, 256))
    f = tmp_path / "model.safetensors"
    _save(f, d)
    f.write_bytes(f.read_bytes()[:-100])
    r = _run("qlinear", tmp_path, tmp_path / "o.bin", "w")
    assert r.returncode == 2 and "outside the" in r.stderr, r.stderr
