"""Parity of the attention layer (dt_attn_layer_fwd: projections, q/k norm, RoPE, flash, o_proj)
with the oracle's OlmoAttention::forward (OlmoAttention.cpp:56-108)."""

import numpy as np
import pytest
import torch

import oracle
from dirktensor_amd import OlmoAttention, synth
from parity import TOL_BF16, TOL_FP32, rel_err, to_np

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def weights():
    return synth.attention_layer_weights()


@pytest.fixture(scope="module")
def layer(gpu, weights):
    w = weights
    return OlmoAttention.from_weights(w["wq"], w["wk"], w["wv"], w["wo"], w["q_norm"], w["k_norm"])


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
def test_config2_layer_t512(gpu, weights, layer, mode):
    """x [1,512,2048] ~ N(0,1) seed 2001; weights ~ N(0,0.02); norms ~ 1+N(0,0.01); theta 5e5."""
    x = synth.layer_input()
    w = weights
    ref = oracle.attention_layer_forward(x, w["wq"], w["wk"], w["wv"], w["wo"], w["q_norm"], w["k_norm"])
    out = layer.forward(torch.from_numpy(x).to(gpu), mode=mode)
    torch.cuda.synchronize()
    err = rel_err(to_np(out), ref)
    print(f"config2 {mode}: rel err {err:.3e}")
    assert err <= (TOL_FP32 if mode == "fp32" else TOL_BF16)


def test_layer_ragged_and_host_path(gpu, weights, layer):
    """A right-padded batch through the host-memory path: valid rows match each sequence run alone."""
    w = weights
    lens = np.array([300, 17, 150], dtype=np.int32)
    x = synth.normal(2101, (3, 300, 2048))
    out = layer.forward(x, seq_lens=lens)
    for b, L in enumerate(lens):
        ref = oracle.attention_layer_forward(x[b:b + 1, :L], w["wq"], w["wk"], w["wv"], w["wo"], w["q_norm"],
                                             w["k_norm"])
        assert rel_err(out[b, :L], ref[0]) <= TOL_FP32


def test_load_from_npy_folder(gpu, weights, layer, tmp_path):
    """OlmoAttention(folder, index) reads the reference's per-layer .npy files (OlmoAttention.cpp:39-53)."""
    names = dict(wq="q_proj", wk="k_proj", wv="v_proj", wo="o_proj", q_norm="q_norm", k_norm="k_norm")
    for key, n in names.items():
        np.save(tmp_path / f"model.layers.3.self_attn.{n}.weight.npy", weights[key])
    loaded = OlmoAttention(str(tmp_path), 3)
    x = torch.from_numpy(synth.normal(2201, (1, 64, 2048))).to(gpu)
    a = loaded.forward(x)
    b = layer.forward(x)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
