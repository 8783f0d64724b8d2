"""The oracle and the seeded generators against the committed golden fixtures (CPU only)."""

import os

import numpy as np
import torch

import oracle
from dirktensor_amd import synth

G = os.path.join(os.path.dirname(__file__), "golden")
SCALE = float(np.float32(1.0) / np.sqrt(np.float32(128.0)))


def load(name):
    return np.load(os.path.join(G, name))


def test_synth_fixture():
    g = load("synth_checks.npz")
    assert np.array_equal(synth.splitmix64(1001, 8), g["splitmix_seed1001"])
    assert np.array_equal(synth.normal(1001, (16,)), g["normal_seed1001"])
    assert np.array_equal(synth.ragged_lengths(), g["lengths_seed4001"])


def test_splitmix_known_answer():
    # splitmix64 with state 0: the published first output of the generator
    assert int(synth.splitmix64(0, 1)[0]) == 0xE220A8397B1DCDAF


def test_synth_statistics_and_bf16_rounding():
    x = synth.normal(1234, (200000,))
    assert abs(float(x.mean())) < 0.01 and abs(float(x.std()) - 1.0) < 0.01
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(synth.to_bf16_bits(x), ref)
    lens = synth.ragged_lengths()
    assert lens.shape == (8,) and lens.min() >= 64 and lens.max() <= 2048


def test_oracle_flash_config1_fixture():
    g = load("flash_config1_fp32.npz")
    Q, K, V = synth.qkv(1, 64, 16)
    O, m, l = oracle.flash_attention_forward(Q, K, V, SCALE)
    assert np.allclose(O, g["O"], rtol=0, atol=1e-6)
    assert np.allclose(m, g["m"], rtol=0, atol=1e-6) and np.allclose(l, g["l"], rtol=1e-6, atol=0)


def test_oracle_norm_rope_fixture():
    g = load("norm_rope_small.npz")
    w = synth.attention_layer_weights()
    q = synth.normal(601, (1, 8, 2048))
    k = synth.normal(602, (1, 8, 2048))
    s, c = oracle.rope_tables(8)
    qn, q_rms = oracle.rmsnorm_forward(q, w["q_norm"])
    kn, k_rms = oracle.rmsnorm_forward(k, w["k_norm"])
    assert np.allclose(oracle.apply_rope(qn.reshape(1, 8, 16, 128), s, c), g["q_out"], rtol=0, atol=1e-6)
    assert np.allclose(oracle.apply_rope(kn.reshape(1, 8, 16, 128), s, c), g["k_out"], rtol=0, atol=1e-6)
    assert np.allclose(q_rms, g["q_rms"], rtol=1e-6) and np.allclose(k_rms, g["k_rms"], rtol=1e-6)


def test_oracle_layer_fixture():
    g = load("layer_small.npz")
    w = synth.attention_layer_weights()
    x = synth.layer_input(1, 16)
    out = oracle.attention_layer_forward(x, w["wq"], w["wk"], w["wv"], w["wo"], w["q_norm"], w["k_norm"])
    assert np.allclose(out, g["out"], rtol=0, atol=1e-5 * np.max(np.abs(g["out"])))


def test_rope_table_fixture():
    g = load("rope_table_checks.npz")
    s, c = oracle.rope_tables(8192)
    assert np.array_equal(s[g["rows"]], g["sin"]) and np.array_equal(c[g["rows"]], g["cos"])
