"""Parity of the fused q/k RMSNorm + RoPE kernel (dt_qk_norm_rope_fwd) with the oracle's
RMSNorm::forward (RMSNorm.cpp:15-22) followed by apply_rope (OlmoAttention.cpp:111-146)."""

import numpy as np
import pytest
import torch

import oracle
from dirktensor_amd import qk_norm_rope, synth
from parity import rel_err, to_np

pytestmark = pytest.mark.gpu

TOL = 2e-6  # fp32 elementwise work: a few ulps of max|out|
TOL_BF16_OUT = 2.0 ** -8


def oracle_norm_rope(q, k, qw, kw):
    B, T, dm = q.shape
    H = dm // 128
    s, c = oracle.rope_tables(max(T, 1))
    qn, q_rms = oracle.rmsnorm_forward(q, qw)
    kn, k_rms = oracle.rmsnorm_forward(k, kw)
    qr = oracle.apply_rope(qn.reshape(B, T, H, 128), s, c)
    kr = oracle.apply_rope(kn.reshape(B, T, H, 128), s, c)
    return qr, kr, q_rms, k_rms


@pytest.mark.parametrize("B,T", [(1, 512), (2, 37), (1, 8192)])
def test_fp32_out(gpu, B, T):
    q = synth.normal(501, (B, T, 2048), 0.0, 3.0)
    k = synth.normal(502, (B, T, 2048), 0.0, 0.5)
    w = synth.attention_layer_weights()
    qr, kr, q_rms, k_rms = oracle_norm_rope(q, k, w["q_norm"], w["k_norm"])
    tq, tk = (torch.from_numpy(x).to(gpu) for x in (q, k))
    tw = [torch.from_numpy(w[n]).to(gpu) for n in ("q_norm", "k_norm")]
    gq, gk, grq, grk = qk_norm_rope(tq, tk, tw[0], tw[1], return_rms=True)
    torch.cuda.synchronize()
    assert rel_err(to_np(gq), qr) <= TOL
    assert rel_err(to_np(gk), kr) <= TOL
    assert rel_err(to_np(grq), q_rms) <= TOL and rel_err(to_np(grk), k_rms) <= TOL


def test_bf16_out(gpu):
    q = synth.normal(511, (1, 300, 2048))
    k = synth.normal(512, (1, 300, 2048))
    w = synth.attention_layer_weights()
    qr, kr, _, _ = oracle_norm_rope(q, k, w["q_norm"], w["k_norm"])
    gq, gk = qk_norm_rope(torch.from_numpy(q).to(gpu), torch.from_numpy(k).to(gpu),
                          torch.from_numpy(w["q_norm"]).to(gpu), torch.from_numpy(w["k_norm"]).to(gpu),
                          out_dtype="bf16")
    torch.cuda.synchronize()
    assert gq.dtype == torch.bfloat16
    assert rel_err(to_np(gq), qr) <= TOL_BF16_OUT
    assert rel_err(to_np(gk), kr) <= TOL_BF16_OUT


def test_host_path_and_position_zero(gpu):
    """numpy (host-memory) path; at t = 0 RoPE is the identity, so the output is the plain RMSNorm."""
    q = synth.normal(521, (3, 5, 2048))
    k = synth.normal(522, (3, 5, 2048))
    qw = np.ones(2048, np.float32)
    kw = synth.normal(523, (2048,), 1.0, 0.01)
    gq, gk = qk_norm_rope(q, k, qw, kw)
    qr, kr, _, _ = oracle_norm_rope(q, k, qw, kw)
    assert rel_err(gq, qr) <= TOL and rel_err(gk, kr) <= TOL
    qn, _ = oracle.rmsnorm_forward(q, qw)
    assert rel_err(gq[:, 0].reshape(3, 2048), qn[:, 0]) <= TOL
