"""Parity of the attention layer's training path (dt_attn_layer_fwd with save_for_backward,
dt_attn_layer_bwd, _step, _zero_grad) with the oracle's OlmoAttention::backward
(OlmoAttention.cpp:193-312), which is pinned against torch autograd through HF's
Olmo2Attention in test_oracle_pins.py.

Checked per result: d_x and the six accumulated parameter gradients, err =
max|got - ref| / max|ref| <= 1e-4 (fp32 exact mode) or 2e-2 (bf16 mode).
"""

import numpy as np
import pytest
import torch

import oracle
from dirktensor_amd import OlmoAttention, synth
from parity import TOL_BF16, TOL_FP32, rel_err, to_np

pytestmark = pytest.mark.gpu

KEYS = ("wq", "wk", "wv", "wo", "q_norm", "k_norm")


@pytest.fixture(scope="module")
def weights():
    return synth.attention_layer_weights()


def new_layer(w):
    return OlmoAttention.from_weights(*(w[k] for k in KEYS))


def run(layer, x, g, dev, mode):
    out = layer.forward(torch.from_numpy(x).to(dev), mode=mode)
    dx = layer.backward(torch.from_numpy(g).to(dev))
    torch.cuda.synchronize()
    return to_np(out), to_np(dx)


@pytest.mark.parametrize("mode,B,T", [("fp32", 1, 64), ("fp32", 2, 40), ("fp32", 1, 200), ("bf16", 1, 128),
                                      ("bf16", 2, 96)])
def test_layer_backward(gpu, weights, mode, B, T):
    w = weights
    x = synth.normal(2501 + T, (B, T, 2048))
    g = synth.normal(2502 + T, (B, T, 2048))
    ref_dx, ref_g = oracle.attention_layer_backward(x, *(w[k] for k in KEYS), g)
    layer = new_layer(w)
    _, dx = run(layer, x, g, gpu, mode)
    grads = layer.grads()
    tol = TOL_FP32 if mode == "fp32" else TOL_BF16
    errs = {"d_x": rel_err(dx, ref_dx)}
    errs.update({k: rel_err(grads[k], ref_g[k]) for k in KEYS})
    print(f"{mode} B={B} T={T}: " + " ".join(f"{k} {v:.2e}" for k, v in errs.items()))
    assert max(errs.values()) <= tol, errs


def test_config2_layer_backward_t512(gpu, weights):
    """x [1,512,2048] seed 2001 (the layer workload) with dL/dout ~ N(0,1) seed 2002, fp32 exact mode."""
    w = weights
    x = synth.layer_input()
    g = synth.normal(2002, x.shape)
    ref_dx, ref_g = oracle.attention_layer_backward(x, *(w[k] for k in KEYS), g)
    layer = new_layer(w)
    _, dx = run(layer, x, g, gpu, "fp32")
    grads = layer.grads()
    assert rel_err(dx, ref_dx) <= TOL_FP32
    for k in KEYS:
        assert rel_err(grads[k], ref_g[k]) <= TOL_FP32, k


def test_grads_accumulate_until_zero_grad(gpu, weights):
    """param<2>::grad semantics: backward adds (beta = 1), zero_grad clears (OlmoAttention.cpp:323-330)."""
    x = synth.normal(2601, (1, 48, 2048))
    g = synth.normal(2602, (1, 48, 2048))
    layer = new_layer(weights)
    run(layer, x, g, gpu, "fp32")
    once = layer.grads()
    run(layer, x, g, gpu, "fp32")
    twice = layer.grads()
    for k in KEYS:
        assert rel_err(twice[k], 2.0 * once[k]) <= 1e-6, k
    layer.zero_grad()
    assert all(np.count_nonzero(v) == 0 for v in layer.grads().values())


@pytest.mark.parametrize("mode,tol", [("fp32", 1e-6), ("bf16", 1e-4)])
def test_backward_after_zero_grad_overwrites(gpu, weights, mode, tol):
    """zero_grad leaves the buffers as they are and the next backward writes the gradients instead of adding
    to them: after backward(x1), zero_grad, backward(x2) the gradients are those of x2 alone (the gradients
    of a new layer's single backward on x2; the GEMMs then differ only in beta, so the tolerance is tight),
    a further backward adds to them again, and a step right after zero_grad leaves the weights unchanged."""
    x1, g1 = synth.normal(2611, (1, 64, 2048)), synth.normal(2612, (1, 64, 2048))
    x2, g2 = synth.normal(2613, (1, 64, 2048)), synth.normal(2614, (1, 64, 2048))
    ref = new_layer(weights)
    run(ref, x2, g2, gpu, mode)
    only2 = ref.grads()
    run(ref, x1, g1, gpu, mode)
    both = ref.grads()
    layer = new_layer(weights)
    run(layer, x1, g1, gpu, mode)
    layer.zero_grad()
    run(layer, x2, g2, gpu, mode)  # no read of the gradients between zero_grad and this backward
    run(layer, x1, g1, gpu, mode)
    got = layer.grads()
    for k in KEYS:
        assert rel_err(got[k], both[k]) <= tol, k
    layer.zero_grad()
    run(layer, x2, g2, gpu, mode)
    got = layer.grads()
    for k in KEYS:
        assert rel_err(got[k], only2[k]) <= tol, k
    layer.zero_grad()
    w0 = layer.weights()
    layer.step(0.5)
    w1 = layer.weights()
    assert all(np.array_equal(w0[k], w1[k]) for k in KEYS)
    assert all(np.count_nonzero(v) == 0 for v in layer.grads().values())


def test_step_is_sgd(gpu, weights):
    """step(lr): w -= lr * grad for all six parameters (OlmoAttention.cpp:314-321), then forward uses them."""
    x = synth.normal(2701, (1, 32, 2048))
    g = synth.normal(2702, (1, 32, 2048))
    layer = new_layer(weights)
    for mode in ("bf16", "fp32"):  # a bf16 forward first: its weight copies must follow the update
        layer.zero_grad()
        run(layer, x, g, gpu, mode)
        before, grads = layer.weights(), layer.grads()
        layer.step(0.01)
        after = layer.weights()
        for k in KEYS:
            expect = before[k] - np.float32(0.01) * grads[k]  # fp32 product, then fp32 difference
            diff = np.abs(after[k].astype(np.float64) - expect)
            assert diff.max() == 0.0, f"{k}: {int(np.count_nonzero(diff))} entries differ, max {diff.max():.3e}"
    w2 = layer.weights()
    ref = oracle.attention_layer_forward(x, *(w2[k] for k in KEYS))
    out = layer.forward(x, mode="bf16")
    assert rel_err(out, ref) <= TOL_BF16


def test_backward_needs_a_saved_forward(gpu, weights):
    from dirktensor_amd import DTError

    layer = new_layer(weights)
    x = torch.from_numpy(synth.normal(2801, (1, 16, 2048))).to(gpu)
    layer.forward(x, save_for_backward=False)
    with pytest.raises(DTError, match="save_for_backward"):
        layer.backward(x)
    layer.forward(x)
    with pytest.raises(DTError, match="differ"):
        layer.backward(torch.zeros((1, 17, 2048), device=gpu))


@pytest.mark.parametrize("mode,B,T", [("bf16", 1, 128), ("bf16", 2, 96), ("bf16", 1, 300), ("fp32", 1, 200),
                                      ("fp32", 2, 40)])
def test_layer_backward_ds_path(gpu, weights, mode, B, T):
    """Layer backward with the attention core's dQ formed from the stored dS (DT_BWD_DQ_FROM_DS)."""
    from dirktensor_amd import Context

    ctx = Context(0)
    ctx.set_bwd_dq_path("from_ds")
    w = weights
    x = synth.normal(2501 + T, (B, T, 2048))
    g = synth.normal(2502 + T, (B, T, 2048))
    ref_dx, ref_g = oracle.attention_layer_backward(x, *(w[k] for k in KEYS), g)
    layer = OlmoAttention.from_weights(*(w[k] for k in KEYS), ctx=ctx)
    _, dx = run(layer, x, g, gpu, mode)
    grads = layer.grads()
    errs = {"d_x": rel_err(dx, ref_dx)}
    errs.update({k: rel_err(grads[k], ref_g[k]) for k in KEYS})
    print(f"dS path {mode} B={B} T={T}: " + " ".join(f"{k} {v:.2e}" for k, v in errs.items()))
    assert max(errs.values()) <= (TOL_FP32 if mode == "fp32" else TOL_BF16), errs
