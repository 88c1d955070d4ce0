"""Runs the C++ test programs (tests/cpp/*.cpp, built by __graft_entry__.build())
that exercise the C++ operator surface (namespace minicpmv) the way the
reference's own tests exercise theirs: standalone programs, non-zero exit on
failure."""
import os
import subprocess
from pathlib import Path

import pytest

BIN = Path(__file__).resolve().parent / "cpp" / "bin"


def run(name, *args, env=None, timeout=120):
    exe = BIN / name
    if not exe.exists():
        pytest.fail(f"{exe} not built (run __graft_entry__.build())")
    e = dict(os.environ)
    e.pop("MINICPM_W8A8_DECODE", None)
    if env:
        e.update(env)
    p = subprocess.run([str(exe), *args], capture_output=True, text=True, timeout=timeout, env=e)
    print(p.stdout, p.stderr)
    assert p.returncode == 0, f"{name} exited {p.returncode}\n{p.stdout}\n{p.stderr}"
    return p.stdout


def test_safetensors_index(tmp_path):
    out = run("test_weights_safetensors", str(tmp_path))
    assert out.strip().endswith("ok")


POLICY = {
    # value -> (layers, enabled, allowed tokens)
    None: (0, 0, set()),
    "": (1, 0, set()),                        # decoder_layer.cpp treats an empty string as enabled
    "0": (0, 0, set()),
    "false": (0, 0, set()),
    "1": (1, 1, {"lm_head"}),
    "selective": (1, 1, {"lm_head"}),
    "all": (1, 1, {"mlp", "linear_qkv", "linear_z", "linear_out", "full_q", "full_k", "full_v", "full_o", "lm_head"}),
    "mlp,full_o": (1, 1, {"mlp", "full_o"}),
}


@pytest.mark.parametrize("value", list(POLICY), ids=lambda v: repr(v))
def test_w8a8_policy(value):
    env = {} if value is None else {"MINICPM_W8A8_DECODE": value}
    out = run("test_decode_dispatch", "policy", env=env).split()
    kv = dict(x.split("=") for x in out)
    layers, enabled, allowed = POLICY[value]
    assert int(kv.pop("layers")) == layers and int(kv.pop("enabled")) == enabled
    assert {k for k, v in kv.items() if v == "1"} == allowed


@pytest.mark.gpu
def test_cpp_matmul_w4a16():
    run("test_matmul_w4a16")


@pytest.mark.gpu
def test_cpp_matmul_w8a8_i32():
    run("test_matmul_w8a8_i32")


@pytest.mark.gpu
def test_cpp_w8a8_dequant(tmp_path):
    """The reference's deterministic dequant vectors (the committed fixture)
    through the C++ surface, as raw files the program reads."""
    import numpy as np
    g = np.load(Path(__file__).resolve().parent / "golden" / "w8a8_dequant_reference.npz")
    g["acc"].reshape(-1).astype("<i4").tofile(tmp_path / "acc.i32")
    g["ws16"].reshape(-1).astype("<u2").tofile(tmp_path / "ws.f16")
    g["xs16"].reshape(-1).astype("<u2").tofile(tmp_path / "xs.f16")
    g["out16"].reshape(-1).astype("<u2").tofile(tmp_path / "out.f16")
    out = run("test_w8a8_dequant", str(tmp_path))
    assert out.strip().endswith("ok")


@pytest.mark.gpu
def test_cpp_quantized_weight_load(tmp_path):
    run("test_quantized_weight_load", str(tmp_path))


@pytest.mark.gpu
def test_cpp_lm_head():
    run("test_lm_head_w4a16")


@pytest.mark.gpu
@pytest.mark.timeout(400)
def test_cpp_lm_head_from_embedding(tmp_path):
    """load_lm_head_w4a16 / _w8a8 over a synthetic [248094, 1024] embedding in a
    safetensors file, through lm_head_greedy_w4a16 / _w8a8, against the oracle."""
    run("test_lm_head_embedding", str(tmp_path), timeout=360)


@pytest.mark.gpu
@pytest.mark.parametrize("mode", [None, "all"])
def test_cpp_decode_dispatch(mode):
    run("test_decode_dispatch", "dispatch", env={} if mode is None else {"MINICPM_W8A8_DECODE": mode})
