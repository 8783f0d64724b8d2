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


# 1000: rows held in registers; 999: the scalar row path; 102404: rows too long for registers, two float4 passes
@pytest.mark.parametrize("on_device,V", [(True, 1000), (False, 1000), (True, 999), (True, 102404)])
def test_ce_loss_and_gradient(gpu, on_device, V):
    B, T = (3, 70) if V < 10000 else (3, 9)
    logits = synth.normal(6201, (B, T, V), 0.0, 3.0)
    tok = synth.model_tokens(B, T, V, seed=6202)
    tok[1, 40:] = PAD  # right padding (main.cpp:46-57)
    tok[2, 7] = PAD
    ref_loss, ref_g = oracle.ce_loss(logits, tok, PAD, with_grad=True)
    src = torch.from_numpy(logits).to(gpu) if on_device else logits
    loss, g = ce_loss(src, tok, PAD, with_grad=True)
    # (the two-pass path's per-thread sums run over 400 terms: fp32 rounding of sum exp reaches ~3e-5 there)
    tol = 1e-5 if V < 10000 else 1e-4
    assert abs(loss - ref_loss) <= tol * abs(ref_loss)
    assert rel_err(to_np(g), ref_g) <= tol
    assert ce_loss(src, tok, PAD) == loss


@pytest.mark.parametrize("V", [1000, 999, 102404])
def test_ce_loss_gradient_in_place(gpu, V):
    """d_logits == logits, as main.cpp reuses probs for the gradient (main.cpp:62-80): same loss and gradient
    as with separate buffers."""
    from dirktensor_amd import _capi, default_context

    B, T = 2, 33
    logits = synth.normal(6211, (B, T, V), 0.0, 3.0)
    tok = synth.model_tokens(B, T, V, seed=6212)
    tok[0, 20:] = PAD
    ref_loss, ref_g = oracle.ce_loss(logits, tok, PAD, with_grad=True)
    buf = torch.from_numpy(logits).to(gpu)
    loss = np.zeros(1, np.float32)
    tok32 = np.ascontiguousarray(tok, np.int32)
    _capi.call("dt_ce_loss", default_context(0).handle, buf.data_ptr(), tok32.ctypes.data, B, T, V, PAD,
               loss.ctypes.data, buf.data_ptr(), _capi.DT_MEM_DEVICE, torch.cuda.current_stream().cuda_stream)
    tol = 1e-5 if V < 10000 else 1e-4  # as in test_ce_loss_and_gradient
    assert abs(float(loss[0]) - ref_loss) <= tol * abs(ref_loss)
    assert rel_err(to_np(buf), ref_g) <= tol


def test_ce_loss_without_targets_is_nan(gpu):
    """Every next token ignored: the reference's 0 / 0 (CrossEntropyLoss.cpp:40, main.cpp:88), NaN loss and
    gradient, like the oracle."""
    V = 64
    logits = synth.normal(6221, (2, 9, V))
    tok = np.full((2, 9), PAD, np.int32)
    tok[:, 0] = 3
    loss, g = ce_loss(torch.from_numpy(logits).to(gpu), tok, PAD, with_grad=True)
    assert np.isnan(loss) and bool(torch.isnan(g).all())


def test_model_loss_full_vocab_shape(gpu):
    """ce_loss over the reference's vocab width (100352 logits per row) on a short sequence."""
    V = 100352
    logits = synth.normal(6301, (1, 12, V), 0.0, 2.0)
    tok = synth.model_tokens(1, 12, V, seed=6302)
    ref = oracle.ce_loss(logits, tok, 100277)
    assert abs(ce_loss(torch.from_numpy(logits).to(gpu), tok, 100277) - ref) <= 1e-5 * abs(ref)


@pytest.mark.parametrize("mode,tol", [("fp32", TOL_FP32), ("bf16", TOL_BF16)])
def test_model_backward(gpu, params, mode, tol):
    """OlmoModel::backward (OlmoModel.cpp:50-67): every parameter gradient against the oracle."""
    B, T = 1, 48
    tok = synth.model_tokens(B, T, VOCAB, seed=6401)
    G = synth.normal(6402, (B, T, VOCAB), 0.0, 1e-3)
    ref = oracle.model_backward(tok, params, G)
    model = OlmoModel.from_params(params)
    model.forward(tok, mode=mode)
    model.backward(torch.from_numpy(G).to(gpu))
    errs = {k: rel_err(model.grad(k), ref[k]) for k in params}
    worst = sorted(errs.items(), key=lambda kv: -kv[1])[:4]
    print(f"model backward {mode}: worst " + ", ".join(f"{k} {v:.2e}" for k, v in worst))
    assert max(errs.values()) <= tol, worst


@pytest.mark.parametrize("mode,tol", [("fp32", 1e-6), ("bf16", 1e-4)])
def test_backward_after_zero_grad_overwrites(gpu, params, mode, tol):
    """zero_grad clears the embedding gradient at once and defers the others: the next backward writes them
    instead of adding to them. backward(t1), zero_grad, backward(t2), backward(t1) equals a new model's
    backward(t2) then backward(t1) (the GEMMs differ only in beta, so the tolerance is tight); a step right
    after zero_grad leaves the weights unchanged."""
    B, T = 1, 40
    t1, t2 = synth.model_tokens(B, T, VOCAB, seed=6451), synth.model_tokens(B, T, VOCAB, seed=6452)
    G1 = torch.from_numpy(synth.normal(6453, (B, T, VOCAB), 0.0, 1e-3)).to(gpu)
    G2 = torch.from_numpy(synth.normal(6454, (B, T, VOCAB), 0.0, 1e-3)).to(gpu)
    ref = OlmoModel.from_params(params)
    for t, G in ((t2, G2), (t1, G1)):
        ref.forward(t, mode=mode)
        ref.backward(G)
    want = {k: ref.grad(k) for k in params}
    model = OlmoModel.from_params(params)
    model.forward(t1, mode=mode)
    model.backward(G1)
    model.zero_grad()
    for t, G in ((t2, G2), (t1, G1)):  # no read of the gradients in between
        model.forward(t, mode=mode)
        model.backward(G)
    errs = {k: rel_err(model.grad(k), want[k]) for k in params}
    assert max(errs.values()) <= tol, sorted(errs.items(), key=lambda kv: -kv[1])[:3]
    model.zero_grad()
    w0 = {k: model.param(k) for k in params}
    model.step(0.5)
    assert all(np.array_equal(model.param(k), w0[k]) for k in params)
    assert all(np.count_nonzero(model.grad(k)) == 0 for k in params)


@pytest.mark.parametrize("B,T,lr", [(1, 40, 1e-2), (1, 40, 0.0), (1, 40, -1e-2), (2, 100, 1e-2)])
def test_embedding_step_and_zero_grad(gpu, params, B, T, lr):
    """step and zero_grad visit only the embedding rows a backward wrote (up to vocab / 8 distinct rows and
    lr >= +0; the dense passes otherwise): the updated table is w - lr * grad on every row, bit for bit, over
    two backward calls (rows of both batches), and zero_grad leaves the whole gradient zero."""
    model = OlmoModel.from_params(params)
    for seed in (6461, 6462):
        tok = synth.model_tokens(B, T, VOCAB, seed=seed)
        model.forward(tok, mode="fp32")
        model.backward(torch.from_numpy(synth.normal(seed + 10, (B, T, VOCAB), 0.0, 1e-3)).to(gpu))
    key = "model.embed_tokens.weight"
    w, g = model.param(key), model.grad(key)
    assert np.count_nonzero(np.abs(g).sum(axis=1)) > 0
    model.step(lr)
    assert np.array_equal(model.param(key), w - np.float32(lr) * g)
    model.zero_grad()
    assert np.count_nonzero(model.grad(key)) == 0


def test_train_step_like_main_cpp(gpu, params):
    """main.cpp:59-91: forward, ce_loss, its gradient, backward, step(1e-4), zero_grad, forward again; a
    right-padded batch (pad = the ignore index). Losses and updated weights against the oracle."""
    B, T, lr = 2, 40, 1e-4
    tok = synth.model_tokens(B, T, VOCAB, seed=6501)
    tok[1, 30:] = PAD
    model = OlmoModel.from_params(params)
    logits = model.forward(tok, mode="fp32")
    loss1, g = ce_loss(logits, tok, PAD, with_grad=True)
    ref_logits = oracle.model_forward(tok, params)
    ref_loss1, ref_g = oracle.ce_loss(ref_logits, tok, PAD, with_grad=True)
    assert abs(loss1 - ref_loss1) <= 1e-4 * abs(ref_loss1)
    model.backward(g)
    grads = {k: model.grad(k) for k in params}
    ref_grads = oracle.model_backward(tok, params, ref_g)
    for k in params:
        assert rel_err(grads[k], ref_grads[k]) <= TOL_FP32, k
    before = {k: model.param(k) for k in ("lm_head.weight", "model.layers.1.mlp.down_proj.weight",
                                          "model.layers.0.self_attn.q_norm.weight", "model.embed_tokens.weight")}
    model.step(lr)
    for k, w in before.items():
        expect = w - np.float32(lr) * grads[k]
        assert np.array_equal(model.param(k), expect), k
    model.zero_grad()
    assert all(np.count_nonzero(model.grad(k)) == 0 for k in ("lm_head.weight", "model.layers.0.mlp.up_proj.weight"))
    loss2 = ce_loss(model.forward(tok, mode="fp32"), tok, PAD)
    updated = {k: model.param(k) for k in params}
    ref_loss2 = oracle.ce_loss(oracle.model_forward(tok, updated), tok, PAD)
    print(f"loss {loss1:.6f} -> {loss2:.6f} (oracle {ref_loss1:.6f} -> {ref_loss2:.6f})")
    assert abs(loss2 - ref_loss2) <= 1e-4 * abs(ref_loss2)
    assert loss2 < loss1


def test_bf16_forward_after_step(gpu, params):
    """After step(), the bf16 mode's weight copies (refreshed by the SGD pass itself) match the updated fp32
    weights: a bf16 forward of the stepped model against the oracle on the updated parameters."""
    B, T, lr = 1, 48, 1e-2
    tok = synth.model_tokens(B, T, VOCAB, seed=6601)
    model = OlmoModel.from_params(params)
    model.forward(tok, mode="bf16")  # makes the bf16 copies
    G = synth.normal(6602, (B, T, VOCAB), 0.0, 1e-2)
    model.backward(torch.from_numpy(G).to(gpu))
    model.step(lr)
    updated = {k: model.param(k) for k in params}
    assert any(not np.array_equal(updated[k], params[k]) for k in params)
    ref = oracle.model_forward(tok, updated)
    # the step moves the logits far more than the tolerance, so stale copies could not pass
    assert rel_err(ref, oracle.model_forward(tok, params)) > 10 * TOL_BF16
    got = model.forward(tok, mode="bf16", save_for_backward=False)
    err = rel_err(got, ref)
    print(f"bf16 forward after step: rel err {err:.3e}")
    assert err <= TOL_BF16


def test_backward_long_k_products(gpu):
    """bf16 backward of a model whose MLP input gradient (K = 2 * 4096) and LM-head input gradient (K = vocab
    8192) take the split-K path (K >= 4 x max(M, N)): every gradient against the oracle, and bitwise equal over
    two backward passes."""
    vocab, hidden, B, T = 8192, 4096, 1, 16
    p = synth.model_params(1, vocab, hidden, seed_base=6700)
    tok = synth.model_tokens(B, T, vocab, seed=6701)
    G = synth.normal(6702, (B, T, vocab), 0.0, 1e-3)
    ref = oracle.model_backward(tok, p, G)
    runs = []
    for _ in range(2):
        model = OlmoModel.from_params(p)
        model.forward(tok, mode="bf16")
        model.backward(torch.from_numpy(G).to(gpu))
        runs.append({k: model.grad(k) for k in p})
    errs = {k: rel_err(runs[0][k], ref[k]) for k in p}
    worst = sorted(errs.items(), key=lambda kv: -kv[1])[:3]
    print("long-K backward: worst " + ", ".join(f"{k} {v:.2e}" for k, v in worst))
    assert max(errs.values()) <= TOL_BF16, worst
    assert all(np.array_equal(runs[0][k], runs[1][k]) for k in p)


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
def test_side_stream_same_bits(gpu, params, mode):
    """The weight-gradient GEMMs on the context's side stream (the default) give the same bits as everything on
    the caller's stream (DT_OPT_SIDE_STREAM = 0): every gradient after two accumulating backward passes, and
    every parameter after the step that follows."""
    from dirktensor_amd import Context

    B, T = 2, 64
    tok = synth.model_tokens(B, T, VOCAB, seed=6501)
    G = torch.from_numpy(synth.normal(6502, (B, T, VOCAB), 0.0, 1e-3)).to(gpu)
    runs = []
    for side in (True, False):
        ctx = Context(0)
        ctx.set_side_stream(side)
        m = OlmoModel.from_params(params, ctx=ctx)
        for _ in range(2):
            m.forward(tok, mode=mode)
            m.backward(G)
        grads = {k: m.grad(k) for k in params}
        m.step(1e-3)
        runs.append((grads, {k: m.param(k) for k in params}))
        m.close()
        ctx.close()
    for k in params:
        assert np.array_equal(runs[0][0][k], runs[1][0][k]), k
        assert np.array_equal(runs[0][1][k], runs[1][1][k]), k


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
def test_model_load_from_npy_folder(gpu, params, model, mode, tmp_path_factory):
    """OlmoModel(folder) (dt_model_load, OlmoModel.cpp:12-23) reads the reference's .npy files: its logits are
    bit-identical to those of the same parameters set one by one through dt_model_set_param, and every parameter
    reads back exactly."""
    folder = tmp_path_factory.mktemp("olmo_npy")
    for name, arr in params.items():
        np.save(folder / f"{name}.npy", arr)
    loaded = OlmoModel(str(folder), N_LAYERS)
    assert (loaded.n_layers, loaded.d_model, loaded.hidden, loaded.vocab) == (N_LAYERS, 2048, HIDDEN, VOCAB)
    tok = synth.model_tokens(2, 96, VOCAB, seed=6060)
    a = torch.empty((2, 96, VOCAB), dtype=torch.float32, device=gpu)
    b = torch.empty_like(a)
    loaded.forward(tok, mode=mode, save_for_backward=False, out=a)
    model.forward(tok, mode=mode, save_for_backward=False, out=b)
    torch.cuda.synchronize()
    assert torch.isfinite(a).all()
    assert torch.equal(a, b)
    for name in ("model.embed_tokens.weight", "model.layers.1.self_attn.q_norm.weight", "lm_head.weight"):
        assert np.array_equal(loaded.param(name), params[name]), name
    loaded.close()
