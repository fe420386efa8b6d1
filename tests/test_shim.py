"""The C++ operator shim (inferd_amd/csrc/qwen35_ops.h: Qwen35::gemm / Qwen35::encode_moe with the reference's
signatures, engine/src/qwen35.h:1465, 1869) and the device loaders (ckpt_dev.h) through their C++ test program,
tests/cpp/qwen35_ops_test.cpp.

The program is built by tests/cpp/build.py (``__graft_entry__.build()`` runs it)."""
import os
import subprocess

import pytest

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "qwen35_ops_test")


def _need_bin():
    if not os.path.exists(BIN):
        pytest.skip("tests/cpp/qwen35_ops_test is not built (python tests/cpp/build.py)")


def test_gemm_rejects_16bit_like_the_reference():
    """The reference prints the reason and exits with status 1 on a route it cannot take (qwen35.h:1469, 1477)."""
    _need_bin()
    r = subprocess.run([BIN, "--bad-bits"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1, (r.returncode, r.stdout, r.stderr)
    assert "16-bit weights are outside this path" in r.stderr


@pytest.mark.gpu
def test_shim_gemm_and_encode_moe_parity():
    """gemm() on the MLX layout (every mode, flipped, rows_of / kslice_of views) and on the T64 copy, and encode_moe()
    (rmsnorm, bit-exact routing, x += MoE output) against the CPU oracle."""
    assert os.path.exists(BIN), "tests/cpp/qwen35_ops_test is not built"
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0 and "ALL OK" in r.stdout, r.stdout + r.stderr


@pytest.mark.gpu
def test_device_loaders_upload_and_gemm(tmp_path):
    """The device loaders (inferd_amd/csrc/ckpt_dev.h: load_qlinear / load_qlinear_bf16_q8 / load_moe with the
    reference's signatures, weights.h:271-406, moe.h:14-87) upload exactly what the host loader reads, pack the T64
    copy, and gemm() on the loaded layer matches the oracle."""
    import json
    import numpy as np
    from oracle import oracle as orc
    from tests.test_ckpt import _put, _qpart, _save
    assert os.path.exists(BIN), "tests/cpp/qwen35_ops_test is not built"
    rng = np.random.default_rng(11)
    d = {}
    _put(d, "mlp.gate_proj", _qpart(rng, 256, 1024, gs=128))
    _put(d, "mlp.up_proj", _qpart(rng, 256, 1024, gs=128))
    _put(d, "mlp.switch_mlp.gate_proj", _qpart(rng, 64, 256, gs=128, lead=(4,)))
    d["x.weight"] = ("bf16", orc.f32_to_bf16(rng.standard_normal((128, 512)).astype(np.float32)))
    _save(tmp_path / "model.safetensors", d)
    (tmp_path / "config.json").write_text(json.dumps({"quantization": {"bits": 4, "group_size": 128}}))
    r = subprocess.run([BIN, "--ckpt", str(tmp_path)], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0 and "ALL OK" in r.stdout, r.stdout + r.stderr


@pytest.mark.gpu
@pytest.mark.parametrize("T", [1, 16, 128, 2048])
def test_encode_moe_t64_config4_geometry(T):
    """encode_moe on the loader's T64 expert stacks at BASELINE config 4's geometry (H 2048, 512 experts, top-10,
    I 512, the shared expert as expert E of the gathered launches; at one token the decode route streaming the same
    T64 copies): routing indices bit-exact on the GPU's logits, the norm within one bf16 step, and x += MoE(xn)
    against the oracle's composition on 96 tokens spread over the batch."""
    assert os.path.exists(BIN), "tests/cpp/qwen35_ops_test is not built"
    r = subprocess.run([BIN, "--moe-c4", str(T)], capture_output=True, text=True, timeout=600)
    print(r.stdout)
    assert r.returncode == 0 and "ALL OK" in r.stdout, r.stdout + r.stderr
    if T == 1:
        assert "[decode, T64]" in r.stdout and "(shared on T64)" in r.stdout, r.stdout
    else:
        assert "[sorted, T64]" in r.stdout and "(shared = expert E)" in r.stdout, r.stdout
