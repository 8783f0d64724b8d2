"""The C++ drop-in headers (FlashAttention.h / OlmoAttention.h mirrors) on the GPU, driven the way
the reference's callers use them (host tensors in, host tensors out)."""

import os
import subprocess
import sys

import numpy as np
import pytest

import oracle
from dirktensor_amd import synth
from parity import TOL_FP32, rel_err

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SCALE = float(np.float32(1.0) / np.sqrt(np.float32(128.0)))


def exe():
    sys.path.insert(0, os.path.join(ROOT, "tests", "cpp"))
    import build_dropin as cpp_build

    return str(cpp_build.BIN if cpp_build.BIN.exists() else cpp_build.build())


def test_cpp_flash_attention_forward(gpu, tmp_path):
    Q, K, V = synth.qkv(2, 300, 3, seeds=(201, 202, 203))
    for n, a in (("q", Q), ("k", K), ("v", V)):
        a.tofile(tmp_path / f"{n}.f32")
    r = subprocess.run([exe(), "flash", str(tmp_path), "2", "300", "3"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    O = np.fromfile(tmp_path / "o.f32", np.float32).reshape(Q.shape)
    l = np.fromfile(tmp_path / "l.f32", np.float32).reshape(2, 300, 3)
    O_ref, _, l_ref = oracle.flash_attention_forward(Q, K, V, SCALE)
    assert rel_err(O, O_ref) <= TOL_FP32 and rel_err(l, l_ref) <= TOL_FP32


def test_cpp_flash_attention_backward(gpu, tmp_path):
    Q, K, V = synth.qkv(1, 260, 2, seeds=(211, 212, 213))
    G = synth.normal(214, Q.shape)
    O, m, l = oracle.flash_attention_forward(Q, K, V, SCALE)
    for n, a in (("g", G), ("o", O), ("q", Q), ("k", K), ("v", V), ("m", m), ("l", l)):
        a.tofile(tmp_path / f"{n}.f32")
    r = subprocess.run([exe(), "bwd", str(tmp_path), "1", "260", "2"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    ref = oracle.flash_attention_backward(G, O, m, l, Q, K, V, SCALE)
    for n, want in zip(("dq", "dk", "dv"), ref):
        got = np.fromfile(tmp_path / f"{n}.f32", np.float32).reshape(Q.shape)
        assert rel_err(got, want) <= TOL_FP32, n


def test_cpp_olmo_attention_layer(gpu, tmp_path):
    w = synth.attention_layer_weights()
    names = dict(wq="q_proj", wk="k_proj", wv="v_proj", wo="o_proj", q_norm="q_norm", k_norm="k_norm")
    for key, n in names.items():
        np.save(tmp_path / f"model.layers.7.self_attn.{n}.weight.npy", w[key])
    x = synth.normal(2401, (1, 96, 2048))
    g = synth.normal(2402, (1, 96, 2048))
    x.tofile(tmp_path / "x.f32")
    g.tofile(tmp_path / "g.f32")
    r = subprocess.run([exe(), "layer", str(tmp_path), "7", str(tmp_path), "1", "96"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    out = np.fromfile(tmp_path / "out.f32", np.float32).reshape(x.shape)
    ref = oracle.attention_layer_forward(x, w["wq"], w["wk"], w["wv"], w["wo"], w["q_norm"], w["k_norm"])
    assert rel_err(out, ref) <= TOL_FP32
    dx = np.fromfile(tmp_path / "dx.f32", np.float32).reshape(x.shape)
    ref_dx, _ = oracle.attention_layer_backward(x, w["wq"], w["wk"], w["wv"], w["wo"], w["q_norm"], w["k_norm"], g)
    assert rel_err(dx, ref_dx) <= TOL_FP32
