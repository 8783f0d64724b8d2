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


@pytest.fixture(scope="module")
def fused_ctx(gpu):
    """A context whose layer forwards run the fused projection + q/k norm + RoPE kernel."""
    from dirktensor_amd import Context

    ctx = Context(0)
    ctx.set_qkv_path("fused")
    return ctx


@pytest.fixture(scope="module")
def fused_layer(gpu, weights, fused_ctx):
    w = weights
    return OlmoAttention.from_weights(w["wq"], w["wk"], w["wv"], w["wo"], w["q_norm"], w["k_norm"], ctx=fused_ctx)


@pytest.fixture(scope="module")
def gemm_layer(gpu, weights):
    """The same weights on a context whose layer forwards run the library QKV GEMM + the norm/RoPE kernel."""
    from dirktensor_amd import Context

    ctx = Context(0)
    ctx.set_qkv_path("gemm")
    w = weights
    return OlmoAttention.from_weights(w["wq"], w["wk"], w["wv"], w["wo"], w["q_norm"], w["k_norm"], ctx=ctx)


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
@pytest.mark.parametrize("B,T", [(1, 512), (1, 130), (2, 2048)])
def test_fused_qkv_projection(gpu, weights, gemm_layer, fused_layer, mode, B, T):
    """The fused projection + q/k norm + RoPE kernel (OlmoAttention.cpp:63-88) against the oracle and the GEMM
    path; rows not a multiple of the 128-row tile (T=130) and several tile rounds (B*T=4096: 32 row blocks x 48
    tiles on 256 CUs); repeated calls are bit-identical (the per-row sums are added in a fixed order)."""
    x = torch.from_numpy(synth.normal(2301 + T, (B, T, 2048))).to(gpu)
    a = fused_layer.forward(x, mode=mode)
    a2 = fused_layer.forward(x, mode=mode)
    b = gemm_layer.forward(x, mode=mode)
    torch.cuda.synchronize()
    assert torch.isfinite(a).all()
    assert torch.equal(a, a2)
    tol = TOL_FP32 if mode == "fp32" else TOL_BF16
    err = rel_err(to_np(a), to_np(b))
    print(f"fused vs GEMM path {mode} B={B} T={T}: rel err {err:.3e}")
    assert err <= tol
    w = weights
    ref = oracle.attention_layer_forward(to_np(x), w["wq"], w["wk"], w["wv"], w["wo"], w["q_norm"], w["k_norm"])
    err = rel_err(to_np(a), ref)
    print(f"fused {mode} B={B} T={T}: rel err vs oracle {err:.3e}")
    assert err <= tol


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
def test_fused_qkv_wait_gives_up_loudly(gpu, weights, mode):
    """A wait for the other heads' row sums that gives up (forced from the host: a spin limit of 0, so every
    workgroup's wait gives up at once and every kernel still ends normally) writes its q/k rows as NaN (which the
    attention core then turns into its empty rows, so the layer output is wrong) and is reported: dt_ctx_check
    raises DT_ERR_HIP once and clears it, and the synchronous host-memory forward raises too. With the default
    limit restored, the same context computes the oracle's result again."""
    from dirktensor_amd import Context
    from dirktensor_amd import _capi as C

    ctx = Context(0)
    ctx.set_qkv_path("fused")
    w = weights
    lay = OlmoAttention.from_weights(w["wq"], w["wk"], w["wv"], w["wo"], w["q_norm"], w["k_norm"], ctx=ctx)
    x = synth.normal(2351, (1, 256, 2048))
    ctx.check()  # nothing to report yet
    ctx.set_qkv_spin_limit(0)
    ref = oracle.attention_layer_forward(x, w["wq"], w["wk"], w["wv"], w["wo"], w["q_norm"], w["k_norm"])
    out = lay.forward(torch.from_numpy(x).to(gpu), mode=mode)  # device path: stream-ordered, reported later
    torch.cuda.synchronize()
    assert not rel_err(to_np(out), ref) <= 0.5  # (NaN compares false as well)
    with pytest.raises(C.DTError) as e:
        ctx.check()
    assert e.value.code == C.DT_ERR_HIP and "gave up" in str(e.value)
    ctx.check()  # the report was cleared
    with pytest.raises(C.DTError) as e:  # the host-memory path synchronises and reports it itself
        lay.forward(x, mode=mode)
    assert e.value.code == C.DT_ERR_HIP
    ctx.set_qkv_spin_limit(1 << 20)
    good = lay.forward(torch.from_numpy(x).to(gpu), mode=mode)
    ctx.check()
    assert rel_err(to_np(good), ref) <= (TOL_FP32 if mode == "fp32" else TOL_BF16)
    lay.close()
    ctx.close()


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
def test_fused_qkv_saved_state_backward(gpu, weights, fused_layer, mode):
    """The fused forward's saved state (pre-norm q|k, rms, rotated q|k|v) drives the layer backward: d_x and the
    six weight gradients match the oracle's OlmoAttention::backward (OlmoAttention.cpp:193-312) at T=128."""
    w = weights
    x = synth.normal(2401, (1, 128, 2048))
    g = synth.normal(2402, (1, 128, 2048))
    fused_layer.zero_grad()
    fused_layer.forward(torch.from_numpy(x).to(gpu), mode=mode)
    dx = fused_layer.backward(torch.from_numpy(g).to(gpu))
    grads = fused_layer.grads()
    torch.cuda.synchronize()
    ref_dx, ref_g = oracle.attention_layer_backward(x, w["wq"], w["wk"], w["wv"], w["wo"], w["q_norm"], w["k_norm"], g)
    tol = TOL_FP32 if mode == "fp32" else TOL_BF16
    errs = {"dx": rel_err(to_np(dx), ref_dx)}
    for k in ref_g:
        errs[k] = rel_err(to_np(grads[k]), ref_g[k])
    print(f"fused saved state {mode}: " + " ".join(f"{k} {v:.2e}" for k, v in errs.items()))
    assert max(errs.values()) <= tol


def test_gemm_tuning_same_bits_across_contexts(gpu, weights):
    """DT_OPT_GEMM_TUNE (on by default) picks each bf16 GEMM shape's algorithm once per process: two fresh
    contexts give bit-identical bf16 layer forwards through the library GEMMs (QKV N = 6144 and o_proj), at a
    shape no other test has tuned (T = 1536)."""
    from dirktensor_amd import Context

    w = weights
    x = torch.from_numpy(synth.normal(2501, (1, 1536, 2048))).to(gpu)
    outs = []
    for _ in range(2):
        ctx = Context(0)
        ctx.set_qkv_path("gemm")
        lay = OlmoAttention.from_weights(w["wq"], w["wk"], w["wv"], w["wo"], w["q_norm"], w["k_norm"], ctx=ctx)
        outs.append(lay.forward(x, mode="bf16"))
        torch.cuda.synchronize()
        lay.close()
        ctx.close()
    assert torch.isfinite(outs[0]).all()
    assert torch.equal(outs[0], outs[1])
