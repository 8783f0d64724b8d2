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
