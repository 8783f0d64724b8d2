"""Parity metrics shared by the tests.

err = max|O_gpu - O_ref| / max|O_ref| over the compared rows (the tolerance
the reference path is held to: 1e-4 in fp32 exact mode, 2e-2 in bf16 mode).
"""

import numpy as np

TOL_FP32 = 1e-4
TOL_BF16 = 2e-2


def rel_err(got, ref) -> float:
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    scale = np.max(np.abs(ref))
    return float(np.max(np.abs(got - ref)) / (scale if scale > 0 else 1.0))


def to_np(t):
    import torch

    if isinstance(t, torch.Tensor):
        return t.detach().float().cpu().numpy()
    return np.asarray(t)
