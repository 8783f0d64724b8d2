"""dt_flash_attn_bwd_noalloc: the attention-core backward that allocates nothing (its row statistics live in
a fixed per-GPU device array). Through the C ABI, its gradients must equal dt_flash_attn_bwd's bit for bit
(same kernels) on two calls in a row, the second with a smaller input, in both modes; sizes past its limit
are rejected before any HIP call."""


import numpy as np
import pytest

from dirktensor_amd import _capi as C
from dirktensor_amd import synth

SCALE = float(np.float32(1.0) / np.sqrt(np.float32(128.0)))
FAKE = 0x10000  # aligned non-NULL address; never dereferenced because validation fails first


def test_noalloc_rejects_sizes_past_its_scratch():
    # B*T*H = 2 * 8192 * 65 > 2^20 rows: refused with a clear message, before the context is even looked at
    rc = C.lib().dt_flash_attn_bwd_noalloc(None, *([FAKE] * 10), 2, 8192, 65, 128, SCALE, 1, C.DT_BF16, None)
    assert rc == C.DT_ERR_UNSUPPORTED
    assert "no-alloc scratch limit" in C.lib().dt_last_error().decode()


def _inputs(gpu, B, T, H, tdt, seed):
    import torch

    Q = synth.normal(seed, (B, T, H, 128))
    K = synth.normal(seed + 1, (B, T, H, 128))
    V = synth.normal(seed + 2, (B, T, H, 128))
    G = synth.normal(seed + 3, (B, T, H, 128))
    return [torch.from_numpy(x).to(gpu).to(tdt) for x in (Q, K, V, G)]


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["fp32", "bf16"])
def test_noalloc_backward_matches_backward(gpu, mode):
    import torch

    from dirktensor_amd import default_context

    tdt = torch.float32 if mode == "fp32" else torch.bfloat16
    dtype = C.DT_FP32_EXACT if mode == "fp32" else C.DT_BF16
    ctx = default_context(0)
    stream = torch.cuda.current_stream().cuda_stream
    # two calls in a row on the same GPU, the second smaller (the array keeps the first call's statistics)
    for B, T, H, causal, seed in ((2, 300, 4, 1, 7101), (1, 100, 2, 0, 7201)):
        print(f"no-alloc backward {mode}: B={B} T={T} H={H} causal={causal}", flush=True)
        q, k, v, g = _inputs(gpu, B, T, H, tdt, seed)
        o = torch.empty_like(q)
        m = torch.empty((B, T, H), dtype=torch.float32, device=gpu)
        l = torch.empty_like(m)
        C.call("dt_flash_attn_fwd", ctx.handle, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), m.data_ptr(),
               l.data_ptr(), B, T, H, 128, SCALE, causal, None, dtype, C.DT_MEM_DEVICE, stream)
        ref = [torch.empty_like(q) for _ in range(3)]
        got = [torch.full_like(q, float("nan")) for _ in range(3)]
        common = (g.data_ptr(), o.data_ptr(), m.data_ptr(), l.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr())
        C.call("dt_flash_attn_bwd", ctx.handle, *common, *(x.data_ptr() for x in ref), B, T, H, 128, SCALE, causal,
               dtype, C.DT_MEM_DEVICE, stream)
        C.call("dt_flash_attn_bwd_noalloc", ctx.handle, *common, *(x.data_ptr() for x in got), B, T, H, 128, SCALE,
               causal, dtype, stream)
        torch.cuda.synchronize()
        for name, a, b in zip(("dQ", "dK", "dV"), got, ref):
            assert torch.isfinite(b.float()).all()
            assert torch.equal(a, b), f"{name} differs from dt_flash_attn_bwd ({mode}, B={B} T={T} H={H})"


def _bwd_call(fn, ctx, g, o, m, l, q, k, v, outs, B, T, H, causal, dtype, stream, noalloc):
    args = (ctx.handle, g.data_ptr(), o.data_ptr(), m.data_ptr(), l.data_ptr(), q.data_ptr(), k.data_ptr(),
            v.data_ptr(), *(x.data_ptr() for x in outs), B, T, H, 128, SCALE, causal, dtype)
    if noalloc:
        C.call(fn, *args, stream)
    else:
        C.call(fn, *args, C.DT_MEM_DEVICE, stream)


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["fp32", "bf16"])
def test_noalloc_above_the_ds_path_threshold(gpu, mode):
    """B=1 T=4096 H=16 (512 blocks of 128 rows per pass on 256 CUs): the default context's dt_flash_attn_bwd takes
    the dS path there, the no-alloc entry point the recompute path. Bit-identical to a context forced onto the
    recompute path; against the default context dK and dV are bit-identical and dQ agrees within the mode's
    tolerance."""
    import torch

    from dirktensor_amd import Context, default_context

    tdt = torch.float32 if mode == "fp32" else torch.bfloat16
    dtype = C.DT_FP32_EXACT if mode == "fp32" else C.DT_BF16
    B, T, H, causal = 1, 4096, 16, 1
    print(f"no-alloc backward above the dS threshold {mode}: B={B} T={T} H={H}", flush=True)
    rec = Context(0)
    rec.set_bwd_dq_path("recompute")
    dflt = default_context(0)
    stream = torch.cuda.current_stream().cuda_stream
    q, k, v, g = _inputs(gpu, B, T, H, tdt, 7301)
    o = torch.empty_like(q)
    m = torch.empty((B, T, H), dtype=torch.float32, device=gpu)
    l = torch.empty_like(m)
    C.call("dt_flash_attn_fwd", dflt.handle, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), m.data_ptr(),
           l.data_ptr(), B, T, H, 128, SCALE, causal, None, dtype, C.DT_MEM_DEVICE, stream)
    got = [torch.full_like(q, float("nan")) for _ in range(3)]
    ref_rec = [torch.empty_like(q) for _ in range(3)]
    ref_def = [torch.empty_like(q) for _ in range(3)]
    common = (g, o, m, l, q, k, v)
    _bwd_call("dt_flash_attn_bwd_noalloc", rec, *common, got, B, T, H, causal, dtype, stream, True)
    _bwd_call("dt_flash_attn_bwd", rec, *common, ref_rec, B, T, H, causal, dtype, stream, False)
    _bwd_call("dt_flash_attn_bwd", dflt, *common, ref_def, B, T, H, causal, dtype, stream, False)
    torch.cuda.synchronize()
    tol = 1e-4 if mode == "fp32" else 2e-2
    for i, name in enumerate(("dQ", "dK", "dV")):
        assert torch.isfinite(got[i].float()).all()
        assert torch.equal(got[i], ref_rec[i]), f"{name} differs from the recompute-path backward ({mode})"
        if name == "dQ":
            err = float((got[i].float() - ref_def[i].float()).abs().max() / ref_def[i].float().abs().max())
            print(f"  dQ against the default (dS-path) backward: {err:.2e}", flush=True)
            assert err <= tol
        else:
            assert torch.equal(got[i], ref_def[i]), f"{name} differs from the default backward ({mode})"
    rec.close()


@pytest.mark.gpu
def test_noalloc_call_allocates_nothing(gpu):
    """On a fresh context, a no-alloc backward whose row statistics take the whole 8 MiB array (B*T*H = 2^20 rows:
    B=4, T=8192, H=32) leaves the device's free memory unchanged (a warm-up call on a tiny shape loads the kernels
    first), and its gradients are bit-identical to a recompute-path dt_flash_attn_bwd's."""
    import torch

    from dirktensor_amd import Context

    B, T, H, causal = 4, 8192, 32, 1
    print(f"no-alloc backward, free-memory check: B={B} T={T} H={H} bf16", flush=True)
    ctx = Context(0)
    stream = torch.cuda.current_stream().cuda_stream
    q, k, v, g = (torch.randn(B, T, H, 128, device=gpu, generator=torch.Generator(device=gpu).manual_seed(s))
                  .to(torch.bfloat16) for s in (11, 12, 13, 14))
    o = torch.empty_like(q)
    m = torch.empty((B, T, H), dtype=torch.float32, device=gpu)
    l = torch.empty_like(m)
    C.call("dt_flash_attn_fwd", ctx.handle, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), m.data_ptr(),
           l.data_ptr(), B, T, H, 128, SCALE, causal, None, C.DT_BF16, C.DT_MEM_DEVICE, stream)
    got = [torch.empty_like(q) for _ in range(3)]
    small = [x[:1, :64, :2].contiguous() for x in (g, o, q, k, v)]
    sm = m[:1, :64, :2].contiguous()
    sl = l[:1, :64, :2].contiguous()
    souts = [torch.empty_like(small[2]) for _ in range(3)]
    _bwd_call("dt_flash_attn_bwd_noalloc", ctx, small[0], small[1], sm, sl, small[2], small[3], small[4], souts, 1, 64,
              2, causal, C.DT_BF16, stream, True)
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    _bwd_call("dt_flash_attn_bwd_noalloc", ctx, g, o, m, l, q, k, v, got, B, T, H, causal, C.DT_BF16, stream, True)
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0, f"free device memory changed by {free0 - free1} bytes across the no-alloc call"
    ref = [torch.empty_like(q) for _ in range(3)]
    ctx.set_bwd_dq_path("recompute")
    _bwd_call("dt_flash_attn_bwd", ctx, g, o, m, l, q, k, v, ref, B, T, H, causal, C.DT_BF16, stream, False)
    torch.cuda.synchronize()
    for name, a, b in zip(("dQ", "dK", "dV"), got, ref):
        assert torch.isfinite(a.float()).all()
        assert torch.equal(a, b), f"{name} differs from the recompute-path backward"
    ctx.close()
