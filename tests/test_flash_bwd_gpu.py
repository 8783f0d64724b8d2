"""Parity of the HIP attention-core backward (dt_flash_attn_bwd) with the CPU oracle.

The oracle restates flash_attention_backward (FlashAttention.cpp:185-359) and
is pinned in test_oracle_pins.py. Both runs start from the same forward
statistics: the oracle forward on the inputs the GPU sees (fp32, or the
bf16 roundings as fp32), whose O, m and l are handed to both backwards.
Tolerance per gradient (max|g_gpu - g_ref| / max|g_ref|): 1e-4 in fp32 exact
mode, 2e-2 in bf16 mode (bf16 inputs, P and dS rounded to bf16 for the MFMA
products, fp32 accumulation).
"""

import numpy as np
import pytest
import torch

import oracle
from dirktensor_amd import flash_attention_backward, synth
from parity import TOL_BF16, TOL_FP32, rel_err, to_np

pytestmark = pytest.mark.gpu

SCALE = float(np.float32(1.0) / np.sqrt(np.float32(128.0)))


def case(B, T, H, seed, mode, causal=True):
    Q, K, V = synth.qkv(B, T, H, seeds=(seed, seed + 1, seed + 2))
    G = synth.normal(seed + 3, Q.shape)
    if mode == "bf16":
        Q, K, V, G = (synth.round_bf16(x) for x in (Q, K, V, G))
    O, m, l = oracle.flash_attention_forward(Q, K, V, SCALE, causal)
    if mode == "bf16":
        O = synth.round_bf16(O)
    ref = oracle.flash_attention_backward(G, O, m, l, Q, K, V, SCALE, causal)
    return (Q, K, V, G, O, m, l), ref


def gpu_bwd(inputs, dev, mode, causal=True):
    Q, K, V, G, O, m, l = inputs
    tdt = torch.float32 if mode == "fp32" else torch.bfloat16
    q, k, v, g, o = (torch.from_numpy(x).to(dev).to(tdt) for x in (Q, K, V, G, O))
    mm, ll = (torch.from_numpy(x).to(dev) for x in (m, l))
    r = flash_attention_backward(g, o, mm, ll, q, k, v, SCALE, causal)
    torch.cuda.synchronize()
    return to_np(r.d_Q), to_np(r.d_K), to_np(r.d_V)


def check(got, ref, tol, label):
    errs = [rel_err(a, b) for a, b in zip(got, ref)]
    print(f"{label}: rel err dQ {errs[0]:.3e} dK {errs[1]:.3e} dV {errs[2]:.3e}")
    assert all(np.all(np.isfinite(a)) for a in got), "non-finite gradient"
    assert max(errs) <= tol, f"{label}: {errs}"


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
@pytest.mark.parametrize("B,T,H", [(1, 1, 1), (1, 2, 3), (2, 33, 2), (1, 64, 16), (1, 100, 5), (1, 127, 1),
                                   (2, 128, 2), (1, 129, 3), (1, 255, 2), (1, 257, 4), (3, 500, 2), (1, 1000, 1)])
def test_bwd_shapes(gpu, mode, B, T, H):
    inputs, ref = case(B, T, H, 300 + T, mode)
    got = gpu_bwd(inputs, gpu, mode)
    check(got, ref, TOL_FP32 if mode == "fp32" else TOL_BF16, f"{mode} B={B} T={T} H={H}")


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
@pytest.mark.parametrize("T", [1, 64, 129, 300])
def test_bwd_full_attention(gpu, mode, T):
    """causal = false (FlashAttention.cpp:247 skips no block)."""
    inputs, ref = case(2, T, 3, 700 + T, mode, causal=False)
    got = gpu_bwd(inputs, gpu, mode, causal=False)
    check(got, ref, TOL_FP32 if mode == "fp32" else TOL_BF16, f"{mode} full T={T}")


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
@pytest.mark.parametrize("T", [2048, 4096])
def test_bwd_long_context(gpu, mode, T):
    """B=1, H=16, D=128, causal at the long-context sizes: every head against the oracle."""
    inputs, ref = case(1, T, 16, 1001, mode)
    got = gpu_bwd(inputs, gpu, mode)
    check(got, ref, TOL_FP32 if mode == "fp32" else TOL_BF16, f"{mode} T={T}")


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
def test_bwd_row_stochastic_invariants(gpu, mode):
    """Rows of P sum to 1: the keys' dK sum to 0 and the keys' dV sum to the queries' dO sum (per head)."""
    inputs, _ = case(1, 2048, 4, 1101, mode)
    dQ, dK, dV = gpu_bwd(inputs, gpu, mode)
    G = inputs[3].astype(np.float64)
    tol = 1e-4 if mode == "fp32" else 2e-2
    assert np.abs(dK.astype(np.float64).sum(axis=1)).max() <= tol * np.abs(dK).max() * 64
    assert rel_err(dV.astype(np.float64).sum(axis=1), G.sum(axis=1)) <= tol


def test_bwd_host_memory(gpu):
    """numpy in, numpy out (mem = HOST): the reference's synchronous value semantics."""
    (Q, K, V, G, O, m, l), ref = case(1, 200, 2, 1201, "fp32")
    r = flash_attention_backward(G, O, m, l, Q, K, V, SCALE, True)
    check((r.d_Q, r.d_K, r.d_V), ref, TOL_FP32, "host fp32")


def test_bwd_deterministic(gpu):
    """Each gradient row has one owner: two runs agree bit for bit."""
    inputs, _ = case(1, 1000, 4, 1301, "bf16")
    a = gpu_bwd(inputs, gpu, "bf16")
    b = gpu_bwd(inputs, gpu, "bf16")
    assert all(np.array_equal(x, y) for x, y in zip(a, b))


# The dS path (DT_OPT_BWD_DQ = DT_BWD_DQ_FROM_DS): the dK/dV pass stores dS in a context buffer and
# dQ = dS K reads it, on a context that selects it for every shape.
@pytest.fixture(scope="module")
def ds_ctx(gpu):
    from dirktensor_amd import Context

    ctx = Context(0)
    ctx.set_bwd_dq_path("from_ds")
    return ctx


@pytest.fixture(scope="module")
def recompute_ctx(gpu):
    from dirktensor_amd import Context

    ctx = Context(0)
    ctx.set_bwd_dq_path("recompute")
    return ctx


def gpu_bwd_ctx(inputs, ctx, mode, causal=True):
    Q, K, V, G, O, m, l = inputs
    tdt = torch.float32 if mode == "fp32" else torch.bfloat16
    q, k, v, g, o = (torch.from_numpy(x).to("cuda").to(tdt) for x in (Q, K, V, G, O))
    mm, ll = (torch.from_numpy(x).to("cuda") for x in (m, l))
    r = flash_attention_backward(g, o, mm, ll, q, k, v, SCALE, causal, ctx=ctx)
    torch.cuda.synchronize()
    return to_np(r.d_Q), to_np(r.d_K), to_np(r.d_V)


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
@pytest.mark.parametrize("B,T,H", [(1, 1, 1), (1, 2, 3), (2, 33, 2), (1, 64, 16), (1, 100, 5), (1, 127, 1),
                                   (2, 128, 2), (1, 129, 3), (1, 255, 2), (1, 257, 4), (3, 500, 2), (1, 1000, 1)])
def test_bwd_ds_path_shapes(ds_ctx, mode, B, T, H):
    inputs, ref = case(B, T, H, 300 + T, mode)
    check(gpu_bwd_ctx(inputs, ds_ctx, mode), ref, TOL_FP32 if mode == "fp32" else TOL_BF16,
          f"dS path {mode} B={B} T={T} H={H}")


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
@pytest.mark.parametrize("T", [1, 64, 129, 300])
def test_bwd_ds_path_full_attention(ds_ctx, mode, T):
    inputs, ref = case(2, T, 3, 700 + T, mode, causal=False)
    check(gpu_bwd_ctx(inputs, ds_ctx, mode, causal=False), ref, TOL_FP32 if mode == "fp32" else TOL_BF16,
          f"dS path {mode} full T={T}")


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
@pytest.mark.parametrize("T", [2048, 4096])
def test_bwd_ds_path_long_context(ds_ctx, mode, T):
    inputs, ref = case(1, T, 16, 1001, mode)
    check(gpu_bwd_ctx(inputs, ds_ctx, mode), ref, TOL_FP32 if mode == "fp32" else TOL_BF16, f"dS path {mode} T={T}")


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
@pytest.mark.parametrize("B,T,H,causal", [(1, 8192, 2, True), (2, 2000, 3, False)])
def test_bwd_ds_path_max_context(ds_ctx, mode, B, T, H, causal):
    """The longest sequence the API takes (key block 0 sees 128 query tiles, the workspace's largest
    per-head extent) and a long non-causal batch (every key block sees every query tile)."""
    inputs, ref = case(B, T, H, 1701 + T, mode, causal=causal)
    check(gpu_bwd_ctx(inputs, ds_ctx, mode, causal=causal), ref, TOL_FP32 if mode == "fp32" else TOL_BF16,
          f"dS path {mode} B={B} T={T} H={H} causal={causal}")


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
@pytest.mark.parametrize("B,T,H,causal", [(1, 1000, 4, True), (2, 300, 3, False), (1, 4096, 16, True)])
def test_bwd_ds_path_against_recompute(ds_ctx, recompute_ctx, mode, B, T, H, causal):
    """dK and dV come from the same kernel code on both paths (bit-identical); dQ sums the same dS values
    times K (bf16: in another order); the dS path is deterministic like the other."""
    inputs, _ = case(B, T, H, 1401 + T, mode, causal=causal)
    a = gpu_bwd_ctx(inputs, ds_ctx, mode, causal)
    b = gpu_bwd_ctx(inputs, recompute_ctx, mode, causal)
    a2 = gpu_bwd_ctx(inputs, ds_ctx, mode, causal)
    assert all(np.array_equal(x, y) for x, y in zip(a, a2)), "dS path not deterministic"
    assert np.array_equal(a[1], b[1]) and np.array_equal(a[2], b[2]), "dK / dV differ between the paths"
    err = rel_err(a[0], b[0])
    print(f"{mode} B={B} T={T} H={H} causal={causal}: dQ dS path vs recompute {err:.3e}")
    assert err <= (1e-5 if mode == "fp32" else 4e-3)
