"""Parity of the OLMo-2 model on the GPU (dt_model_* and dt_ce_loss) with the oracle's OlmoModel::forward
(OlmoModel.cpp:25-48) and ce_loss (CrossEntropyLoss.cpp:8-43, with main.cpp:62-80's gradient), both pinned
against HF's Olmo2ForCausalLM and torch's cross_entropy in test_oracle_pins.py.

Small models (2 layers, vocab 1000, MLP width 512) at the full d_model = 2048, H = 16; tolerances as for
the attention path: max|got - ref| / max|ref| <= 1e-4 in fp32 exact mode, 2e-2 in bf16 mode.
"""

import numpy as np
import pytest
import torch

import oracle
from dirktensor_amd import OlmoModel, ce_loss, synth
from parity import TOL_BF16, TOL_FP32, rel_err, to_np

pytestmark = pytest.mark.gpu

N_LAYERS, VOCAB, HIDDEN, PAD = 2, 1000, 512, 999


@pytest.fixture(scope="module")
def params():
    return synth.model_params(N_LAYERS, VOCAB, HIDDEN, seed_base=6100)


@pytest.fixture(scope="module")
def model(gpu, params):
    return OlmoModel.from_params(params)


@pytest.mark.parametrize("mode,B,T", [("fp32", 1, 64), ("fp32", 2, 100), ("bf16", 1, 64), ("bf16", 2, 130)])
def test_model_forward(gpu, params, model, mode, B, T):
    tok = synth.model_tokens(B, T, VOCAB, seed=6001 + T)
    ref = oracle.model_forward(tok, params)
    out = torch.empty((B, T, VOCAB), dtype=torch.float32, device=gpu)
    model.forward(tok, mode=mode, save_for_backward=False, out=out)
    torch.cuda.synchronize()
    err = rel_err(to_np(out), ref)
    print(f"model {mode} B={B} T={T}: logits rel err {err:.3e}")
    assert err <= (TOL_FP32 if mode == "fp32" else TOL_BF16)


def test_model_forward_host_memory(gpu, params, model):
    tok = synth.model_tokens(1, 40, VOCAB, seed=6050)
    assert rel_err(model.forward(tok), oracle.model_forward(tok, params)) <= TOL_FP32


def test_params_round_trip(gpu, params, model):
    for name in ("model.embed_tokens.weight", "model.layers.1.mlp.up_proj.weight", "model.layers.0.self_attn.k_proj.weight",
                 "model.layers.1.post_feedforward_layernorm.weight", "lm_head.weight"):
        assert np.array_equal(model.param(name), params[name]), name


@pytest.mark.parametrize("on_device", [True, False])
def test_ce_loss_and_gradient(gpu, on_device):
    B, T, V = 3, 70, 1000
    logits = synth.normal(6201, (B, T, V), 0.0, 3.0)
    tok = synth.model_tokens(B, T, V, seed=6202)
    tok[1, 40:] = PAD  # right padding (main.cpp:46-57)
    tok[2, 7] = PAD
    ref_loss, ref_g = oracle.ce_loss(logits, tok, PAD, with_grad=True)
    src = torch.from_numpy(logits).to(gpu) if on_device else logits
    loss, g = ce_loss(src, tok, PAD, with_grad=True)
    assert abs(loss - ref_loss) <= 1e-5 * abs(ref_loss)
    assert rel_err(to_np(g), ref_g) <= 1e-5
    assert ce_loss(src, tok, PAD) == loss


def test_model_loss_full_vocab_shape(gpu):
    """ce_loss over the reference's vocab width (100352 logits per row) on a short sequence."""
    V = 100352
    logits = synth.normal(6301, (1, 12, V), 0.0, 2.0)
    tok = synth.model_tokens(1, 12, V, seed=6302)
    ref = oracle.ce_loss(logits, tok, 100277)
    assert abs(ce_loss(torch.from_numpy(logits).to(gpu), tok, 100277) - ref) <= 1e-5 * abs(ref)
