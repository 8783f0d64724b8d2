"""Parity of the HIP attention core (dt_flash_attn_fwd) with the CPU oracle.

The oracle restates flash_attention_forward (FlashAttention.cpp:24-182). Tolerances
(max|O_gpu - O_ref| / max|O_ref|): 1e-4 in fp32 exact mode, 2e-2 in bf16 mode,
where the bf16 run sees the RNE-bf16 rounding of the same fp32 draws and is
compared with the oracle on the unrounded fp32 inputs.
"""

import os

import numpy as np
import pytest
import torch

import oracle
from dirktensor_amd import DTError, flash_attention_forward, synth
from parity import TOL_BF16, TOL_FP32, rel_err, to_np

pytestmark = pytest.mark.gpu

SCALE = float(np.float32(1.0) / np.sqrt(np.float32(128.0)))  # 1.0f / sqrtf(128.f), OlmoAttention.cpp:91
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def gpu_flash(Q, K, V, dev, mode, causal=True, seq_lens=None):
    tdt = torch.float32 if mode == "fp32" else torch.bfloat16
    q, k, v = (torch.from_numpy(x).to(dev).to(tdt) for x in (Q, K, V))
    r = flash_attention_forward(q, k, v, SCALE, causal, seq_lens=seq_lens)
    torch.cuda.synchronize()
    return to_np(r.output), to_np(r.softmax_m), to_np(r.softmax_l)


def check_stats(m, l, m_ref, l_ref, tol):
    fin = np.isfinite(m_ref)
    assert np.array_equal(fin, np.isfinite(m)), "m finiteness differs"
    assert np.max(np.abs(m[fin] - m_ref[fin])) <= tol * max(1.0, float(np.max(np.abs(m_ref[fin]))))
    assert rel_err(l, l_ref) <= tol


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
def test_config1_t64(gpu, mode):
    """B=1, T=64, H=16, D=128, causal, Q/K/V ~ N(0,1) seeds 1001-1003."""
    Q, K, V = synth.qkv(1, 64, 16)
    O_ref, m_ref, l_ref = oracle.flash_attention_forward(Q, K, V, SCALE)
    O, m, l = gpu_flash(Q, K, V, gpu, mode)
    tol = TOL_FP32 if mode == "fp32" else TOL_BF16
    err = rel_err(O, O_ref)
    print(f"config1 {mode}: rel err {err:.3e}")
    assert err <= tol
    check_stats(m, l, m_ref, l_ref, tol)


def test_config1_golden(gpu):
    """The GPU fp32 output against the committed oracle fixture (no oracle run needed)."""
    g = np.load(os.path.join(GOLDEN, "flash_config1_fp32.npz"))
    Q, K, V = synth.qkv(1, 64, 16)
    O, m, l = gpu_flash(Q, K, V, gpu, "fp32")
    assert rel_err(O, g["O"]) <= TOL_FP32
    check_stats(m, l, g["m"], g["l"], TOL_FP32)


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
@pytest.mark.parametrize("B,T,H", [(1, 1, 1), (1, 2, 3), (2, 33, 2), (1, 100, 5), (1, 127, 1), (2, 128, 2),
                                   (1, 129, 3), (1, 255, 2), (1, 257, 4), (3, 500, 2), (1, 1000, 1)])
def test_shapes(gpu, mode, B, T, H):
    Q, K, V = synth.qkv(B, T, H, seeds=(11 + T, 12 + T, 13 + T))
    O_ref, m_ref, l_ref = oracle.flash_attention_forward(Q, K, V, SCALE)
    O, m, l = gpu_flash(Q, K, V, gpu, mode)
    tol = TOL_FP32 if mode == "fp32" else TOL_BF16
    assert rel_err(O, O_ref) <= tol
    check_stats(m, l, m_ref, l_ref, tol)


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
@pytest.mark.parametrize("T", [2048, 4096, 6144])
def test_config3_long_context(gpu, mode, T):
    """B=1, H=16, D=128, causal, T in {2048, 4096, 6144}: every head against the oracle."""
    Q, K, V = synth.qkv(1, T, 16)
    O_ref, m_ref, l_ref = oracle.flash_attention_forward(Q, K, V, SCALE)
    O, m, l = gpu_flash(Q, K, V, gpu, mode)
    tol = TOL_FP32 if mode == "fp32" else TOL_BF16
    err = rel_err(O, O_ref)
    print(f"config3 T={T} {mode}: rel err {err:.3e}")
    assert err <= tol
    check_stats(m, l, m_ref, l_ref, tol)


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
def test_non_causal(gpu, mode):
    Q, K, V = synth.qkv(2, 300, 3, seeds=(21, 22, 23))
    O_ref, m_ref, l_ref = oracle.flash_attention_forward(Q, K, V, SCALE, causal=False)
    O, m, l = gpu_flash(Q, K, V, gpu, mode, causal=False)
    tol = TOL_FP32 if mode == "fp32" else TOL_BF16
    assert rel_err(O, O_ref) <= tol
    check_stats(m, l, m_ref, l_ref, tol)


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
def test_config4_ragged(gpu, mode):
    """B=8, lengths ~ U[64, 2048] (seed 4001), right-padded; valid rows against the oracle run on each
    unpadded prefix; padded rows are the reference's empty row (O=0, m=-inf, l=0)."""
    lens = synth.ragged_lengths()
    Tm = int(lens.max())
    Q, K, V = synth.qkv(8, Tm, 16)
    O_ref, m_ref, l_ref = oracle.flash_attention_ragged(Q, K, V, lens, SCALE)
    O, m, l = gpu_flash(Q, K, V, gpu, mode, seq_lens=lens)
    tol = TOL_FP32 if mode == "fp32" else TOL_BF16
    valid = np.arange(Tm)[None, :] < lens[:, None]
    err = rel_err(O[valid], O_ref[valid])
    print(f"config4 lens={lens.tolist()} {mode}: rel err {err:.3e}")
    assert err <= tol
    assert np.all(O[~valid] == 0.0)
    assert np.all(m[~valid] == -np.inf) and np.all(l[~valid] == 0.0)
    check_stats(m[valid], l[valid], m_ref[valid], l_ref[valid], tol)


@pytest.mark.parametrize("B,T,H,lens", [(1, 4096, 2, None), (1, 2048, 4, None), (3, 4096, 2, [4096, 2500, 129]),
                                        (2, 3000, 3, [3000, 2900]), (1, 8192, 2, None)])
def test_split_items(gpu, B, T, H, lens):
    """Shapes whose bf16 schedule splits the longest query tiles' keys across workgroups (up to three parts,
    merged by the last part to finish): against the oracle, and bit-identical on a second call (the merge
    order is fixed and the per-item counters return to zero)."""
    Q, K, V = synth.qkv(B, T, H, seeds=(31 + T, 32 + T, 33 + T))
    if lens is None:
        O_ref, m_ref, l_ref = oracle.flash_attention_forward(Q, K, V, SCALE)
        valid = np.ones((B, T), bool)
    else:
        lens = np.asarray(lens, np.int32)
        O_ref, m_ref, l_ref = oracle.flash_attention_ragged(Q, K, V, lens, SCALE)
        valid = np.arange(T)[None, :] < lens[:, None]
    O, m, l = gpu_flash(Q, K, V, gpu, "bf16", seq_lens=lens)
    assert rel_err(O[valid], O_ref[valid]) <= TOL_BF16
    check_stats(m[valid], l[valid], m_ref[valid], l_ref[valid], TOL_BF16)
    if lens is not None:
        assert np.all(O[~valid] == 0.0) and np.all(m[~valid] == -np.inf) and np.all(l[~valid] == 0.0)
    O2, m2, l2 = gpu_flash(Q, K, V, gpu, "bf16", seq_lens=lens)
    assert np.array_equal(O2, O) and np.array_equal(m2, m) and np.array_equal(l2, l)


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
@pytest.mark.parametrize("B,T,H", [(1, 1024, 16), (2, 2048, 8), (1, 256, 3), (1, 2048, 16)])
def test_folded_launches(gpu, mode, B, T, H):
    """Causal launches of at most one 128-query unit per CU fold their units (64-query tiles p and n-1-p of
    one head per workgroup): against the oracle; causality bit-exact for a row of a lower tile and one of an
    upper tile; and bit-identical to the unfolded schedule, which the same heads take when the launch holds
    copies of its heads beyond one round of a 256-CU part."""
    Q, K, V = synth.qkv(B, T, H, seeds=(41 + T, 42 + T, 43 + T))
    O_ref, m_ref, l_ref = oracle.flash_attention_forward(Q, K, V, SCALE)
    O, m, l = gpu_flash(Q, K, V, gpu, mode)
    tol = TOL_FP32 if mode == "fp32" else TOL_BF16
    err = rel_err(O, O_ref)
    print(f"folded B={B} T={T} H={H} {mode}: rel err {err:.3e}", flush=True)
    assert err <= tol
    check_stats(m, l, m_ref, l_ref, tol)
    for t in (T // 8 + 5, T - T // 16 - 3):
        K2, V2 = K.copy(), V.copy()
        K2[:, t + 1:] = synth.normal(79, K2[:, t + 1:].shape)
        V2[:, t + 1:] = synth.normal(80, V2[:, t + 1:].shape)
        O2, m2, l2 = gpu_flash(Q, K2, V2, gpu, mode)
        assert np.array_equal(O2[:, :t + 1], O[:, :t + 1])
        assert np.array_equal(m2[:, :t + 1], m[:, :t + 1]) and np.array_equal(l2[:, :t + 1], l[:, :t + 1])
    rep = 300 // (B * H * (T // 128)) + 1  # more than 300 units: more than one round on up to 300 CUs
    dup = [np.concatenate([x] * rep, axis=2) for x in (Q, K, V)]
    O3, m3, l3 = gpu_flash(*dup, gpu, mode)
    for r in range(rep):
        part = slice(r * H, (r + 1) * H)
        assert np.array_equal(O3[:, :, part], O) and np.array_equal(m3[:, :, part], m)
        assert np.array_equal(l3[:, :, part], l)


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
def test_properties_full_size(gpu, mode):
    """Size-independent checks at T=4096, H=16: row 0 returns V[0] exactly (one key, p=1, l=1);
    changing K/V after position t leaves rows <= t bit-identical (causality); heads are independent."""
    T = 4096
    Q, K, V = synth.qkv(1, T, 16)
    O, m, l = gpu_flash(Q, K, V, gpu, mode)
    Vin = V if mode == "fp32" else synth.round_bf16(V)
    assert np.array_equal(O[0, 0], Vin[0, 0])
    if mode == "fp32":
        assert np.all(l[0, 0] == 1.0)
    else:
        assert np.max(np.abs(l[0, 0] - 1.0)) <= 1e-5
    t = 2500
    K2, V2 = K.copy(), V.copy()
    K2[:, t + 1:] = synth.normal(77, K2[:, t + 1:].shape)
    V2[:, t + 1:] = synth.normal(78, V2[:, t + 1:].shape)
    O2, m2, l2 = gpu_flash(Q, K2, V2, gpu, mode)
    assert np.array_equal(O2[:, :t + 1], O[:, :t + 1])
    assert np.array_equal(m2[:, :t + 1], m[:, :t + 1]) and np.array_equal(l2[:, :t + 1], l[:, :t + 1])
    perm = np.random.default_rng(0).permutation(16)
    O3, _, _ = gpu_flash(Q[:, :, perm], K[:, :, perm], V[:, :, perm], gpu, mode)
    assert np.array_equal(O3, O[:, :, perm])


def test_host_memory_path(gpu):
    """numpy inputs take the synchronous host-memory path (copy in, compute, copy out)."""
    Q, K, V = synth.qkv(1, 200, 4, seeds=(31, 32, 33))
    r = flash_attention_forward(Q, K, V, SCALE)
    O_ref, m_ref, l_ref = oracle.flash_attention_forward(Q, K, V, SCALE)
    assert isinstance(r.output, np.ndarray)
    assert rel_err(r.output, O_ref) <= TOL_FP32
    check_stats(r.softmax_m, r.softmax_l, m_ref, l_ref, TOL_FP32)


def test_invalid_arguments_raise(gpu):
    q = torch.zeros((1, 16, 2, 64), device=gpu)
    with pytest.raises(DTError):
        flash_attention_forward(q, q, q, SCALE)  # D != 128
    q = torch.zeros((1, 16, 2, 128), device=gpu)
    with pytest.raises(DTError):
        flash_attention_forward(q, q, q, SCALE, seq_lens=[17])  # length > T
