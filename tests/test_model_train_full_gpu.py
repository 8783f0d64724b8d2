"""bf16 training gradients at the full OLMo-2-1B width and a long sequence: a 2-layer model with d_model 2048,
16 heads, MLP width 8192 (vocab 1000 keeps the LM head small), one sequence of T = 2048 tokens, and every
parameter gradient of OlmoModel::backward (OlmoModel.cpp:50-67) against the oracle, with the q/k
RMSNorm-weight gradients (RMSNorm.cpp:24-36, column sums over all 2048 rows) printed. Tolerance: the bf16
bar, max|got - ref| / max|ref| <= 2e-2."""

import pytest
import torch

import oracle
from dirktensor_amd import OlmoModel, synth
from parity import TOL_BF16, rel_err

pytestmark = pytest.mark.gpu

N_LAYERS, VOCAB, HIDDEN, T = 2, 1000, 8192, 2048


def test_model_backward_bf16_full_width_t2048(gpu):
    params = synth.model_params(N_LAYERS, VOCAB, HIDDEN, seed_base=6600)
    tok = synth.model_tokens(1, T, VOCAB, seed=6601)
    G = synth.normal(6602, (1, T, VOCAB), 0.0, 1e-3)
    model = OlmoModel.from_params(params)
    model.forward(tok, mode="bf16")
    model.backward(torch.from_numpy(G).to(gpu))
    torch.cuda.synchronize()
    got = {k: model.grad(k) for k in params}
    del model
    ref = oracle.model_backward(tok, params, G)
    errs = {k: rel_err(got[k], ref[k]) for k in params}
    for k in sorted(errs):
        if "norm" in k:
            print(f"{k}: {errs[k]:.3e}")
    worst = sorted(errs.items(), key=lambda kv: -kv[1])[:4]
    print("worst: " + ", ".join(f"{k} {v:.2e}" for k, v in worst))
    assert max(errs.values()) <= TOL_BF16, worst
