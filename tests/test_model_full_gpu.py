"""The end-to-end workload at its full size: an OLMo-2-1B-shaped forward prefill (OlmoModel::forward,
OlmoModel.cpp:25-48, with the reference's 16 blocks, OlmoModel.cpp:21-22): 16 layers, d_model 2048,
16 heads x 128, SwiGLU MLP 8192, vocab 100352, post-norm RMSNorm eps 1e-6, QK-norm, RoPE 500000, token ids
~ U[0, 100352) from seed 5001, T = 2048, B = 1.

The 1.48 B weights are drawn on the device (synth.device_model_params, seed 5100: matrices ~ N(0, 0.02)
rounded to bf16-representable values, norm weights ~ 1 + N(0, 0.01)) and copied to the host for the
oracle's fp32 OlmoModel::forward (about 6 s on 16 host threads). The logits are compared in both modes:
max|got - ref| / max|ref| <= 2e-2 in bf16 mode and <= 1e-4 in fp32 exact mode.
"""

import os

import numpy as np
import pytest
import torch

import oracle
from dirktensor_amd import OlmoModel, synth
from parity import TOL_BF16, TOL_FP32, rel_err, to_np

pytestmark = pytest.mark.gpu

N_LAYERS, D_MODEL, HIDDEN, VOCAB, T = 16, 2048, 8192, 100352, 2048


def _threads() -> int:
    try:
        return max(1, min(16, len(os.sched_getaffinity(0))))
    except AttributeError:  # pragma: no cover
        return 16


@pytest.fixture(scope="module")
def full(gpu):
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
        _capi.call("dt_model_set_param", model.handle, name.encode(), w.data_ptr(), w.numel(), _capi.DT_MEM_DEVICE)
        host[name] = w.cpu().numpy()
        del w
    tok = synth.model_tokens(1, T, VOCAB)
    print(f"OLMo-2-1B shape: {sum(a.size for a in host.values())} parameters on the device", flush=True)
    ref = oracle.model_forward(tok, host, nthreads=_threads())
    print(f"oracle forward done, max|logit| {np.max(np.abs(ref)):.3f}", flush=True)
    yield model, tok, ref
    model.close()
    host.clear()


@pytest.mark.parametrize("mode,tol", [("bf16", TOL_BF16), ("fp32", TOL_FP32)])
def test_olmo2_1b_forward_full_size(gpu, full, mode, tol):
    model, tok, ref = full
    logits = torch.empty((1, T, VOCAB), dtype=torch.float32, device=gpu)
    model.forward(tok, mode=mode, save_for_backward=False, out=logits)
    torch.cuda.synchronize()
    got = to_np(logits)
    assert np.isfinite(got).all()
    err = rel_err(got, ref)
    # top-1 agreement (the reference's own known-answer test compares top-k token ids, test_olmo_model.cpp:48-70)
    agree = float(np.mean(np.argmax(got[0], axis=-1) == np.argmax(ref[0], axis=-1)))
    print(f"OLMo-2-1B forward {mode}, tokens [1,{T}]: logits rel err {err:.3e} (tol {tol}), "
          f"top-1 agreement {agree:.4f}", flush=True)
    assert err <= tol
