"""main.cpp's training step at the full OLMo-2-1B size (main.cpp:59-93, OlmoModel.cpp:50-75): 16 layers,
d_model 2048, 16 heads x 128, SwiGLU MLP 8192, vocab 100352, one sequence of T = 2048 tokens (~ U[0, 100352)
from seed 5001, the last 48 positions padding = the ignore index, as main.cpp pads a batch).

forward -> ce_loss and its gradient (softmax - onehot) / count -> backward -> step(1e-4) -> zero_grad -> forward
-> ce_loss, in both modes, against the oracle: the first loss and a sample of parameter gradients (q/k norm weights
of the first and last block, where bf16 rounding collects most, projections, the MLP, the final norm, the LM head
and the embedding rows) against the oracle's OlmoModel::backward on the same weights, and the second loss against
the oracle's forward on the weights the GPU step produced. Tolerances: max|got - ref| / max|ref| <= 1e-4 (fp32
exact mode) and <= 2e-2 (bf16 mode) for the gradients; the losses to 1e-4 and 2e-3 relative.

The 1.48 B weights are drawn on the device (synth.device_model_params, seed 5100) and copied to the host for the
oracle (its forward takes about 6 s and its backward about 15 s on 16 host threads).
"""

import os

import numpy as np
import pytest
import torch

import oracle
from dirktensor_amd import OlmoModel, ce_loss, synth
from parity import TOL_BF16, TOL_FP32, rel_err

pytestmark = pytest.mark.gpu

N_LAYERS, D_MODEL, HIDDEN, VOCAB, T, PAD, LR = 16, 2048, 8192, 100352, 2048, 1, 1e-4
SAMPLE = ("model.layers.0.self_attn.q_norm.weight", "model.layers.0.self_attn.k_norm.weight",
          "model.layers.15.self_attn.q_norm.weight", "model.layers.15.self_attn.k_norm.weight",
          "model.layers.0.self_attn.q_proj.weight", "model.layers.7.self_attn.v_proj.weight",
          "model.layers.15.self_attn.o_proj.weight", "model.layers.3.mlp.gate_proj.weight",
          "model.layers.15.mlp.down_proj.weight", "model.layers.8.post_attention_layernorm.weight",
          "model.norm.weight", "lm_head.weight", "model.embed_tokens.weight")


def _threads() -> int:
    try:
        return max(1, min(16, len(os.sched_getaffinity(0))))
    except AttributeError:  # pragma: no cover
        return 16


@pytest.fixture(scope="module")
def setup(gpu):
    import ctypes

    import dirktensor_amd as dt
    from dirktensor_amd import _capi

    ctx = dt.default_context(0)
    h = ctypes.c_void_p()
    _capi.call("dt_model_create", ctx.handle, N_LAYERS, D_MODEL, D_MODEL // 128, HIDDEN, VOCAB, ctypes.byref(h))
    model = OlmoModel(ctx=ctx, _handle=h, _dims=(N_LAYERS, D_MODEL, HIDDEN, VOCAB))
    host = {}
    for name, w in synth.device_model_params(gpu, N_LAYERS, VOCAB, HIDDEN, D_MODEL):
        torch.cuda.synchronize()
        host[name] = w.cpu().numpy()
        del w
    tok = synth.model_tokens(1, T, VOCAB)
    tok[0, T - 48:] = PAD
    nt = _threads()
    print(f"OLMo-2-1B training step: {sum(a.size for a in host.values())} parameters", flush=True)
    ref_logits = oracle.model_forward(tok, host, nthreads=nt)
    ref_loss1, ref_g = oracle.ce_loss(ref_logits, tok, PAD, with_grad=True)
    del ref_logits
    print(f"oracle forward + loss done: loss {ref_loss1:.6f}", flush=True)
    ref_grads = oracle.model_backward(tok, host, ref_g, nthreads=nt)
    ref_grads = {k: ref_grads[k] for k in SAMPLE}
    print("oracle backward done", flush=True)
    yield model, host, tok, ref_loss1, ref_grads
    model.close()
    host.clear()


@pytest.mark.parametrize("mode", ["bf16", "fp32"])
def test_olmo2_1b_train_step_like_main_cpp(gpu, setup, mode):
    model, host, tok, ref_loss1, ref_grads = setup
    for name, w in host.items():  # the initial weights (the other mode's step changed them)
        model.set_param(name, w)
    model.zero_grad()
    logits = torch.empty((1, T, VOCAB), dtype=torch.float32, device=gpu)
    model.forward(tok, mode=mode, out=logits)
    loss1, g = ce_loss(logits, tok, PAD, with_grad=True)
    model.backward(g)
    torch.cuda.synchronize()
    tol = TOL_FP32 if mode == "fp32" else TOL_BF16
    ltol = 1e-4 if mode == "fp32" else 2e-3
    print(f"{mode}: loss {loss1:.6f} (oracle {ref_loss1:.6f})", flush=True)
    assert abs(loss1 - ref_loss1) <= ltol * abs(ref_loss1)
    errs = {k: rel_err(model.grad(k), ref_grads[k]) for k in SAMPLE}
    print(f"{mode} gradients: " + ", ".join(f"{k.replace('model.layers.', 'L')} {v:.2e}" for k, v in errs.items()),
          flush=True)
    assert max(errs.values()) <= tol, max(errs.items(), key=lambda kv: kv[1])
    model.step(LR)
    model.zero_grad()
    model.forward(tok, mode=mode, out=logits)
    loss2 = ce_loss(logits, tok, PAD)
    torch.cuda.synchronize()
    del logits, g
    updated = {k: model.param(k) for k in host}
    assert not np.array_equal(updated["lm_head.weight"], host["lm_head.weight"])
    ref_loss2 = oracle.ce_loss(oracle.model_forward(tok, updated, nthreads=_threads()), tok, PAD)
    del updated
    print(f"{mode}: loss after step {loss2:.6f} (oracle on the stepped weights {ref_loss2:.6f})", flush=True)
    assert abs(loss2 - ref_loss2) <= ltol * abs(ref_loss2)
    assert loss2 < loss1
