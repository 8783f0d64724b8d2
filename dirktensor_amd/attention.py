"""Python mirror of the reference's attention interfaces, on the HIP path.

    flash_attention_forward(Q, K, V, scale, causal=True) -> FlashAttentionResult
        FlashAttention.h:15-21 (returns output, softmax_m, softmax_l,
        FlashAttention.h:6-10)
    flash_attention_backward(dO, O, m, l, Q, K, V, scale, causal=True) -> FlashAttentionGradients
        FlashAttention.h:33-43 (returns d_Q, d_K, d_V, FlashAttention.h:27-31)
    OlmoAttention(folder, index) / OlmoAttention.from_weights(...)
        OlmoAttention.h:10-42; forward(x) -> out
    qk_norm_rope(q_proj, k_proj, q_norm_w, k_norm_w)
        RMSNorm::forward (RMSNorm.cpp:15-22) for q_norm/k_norm + apply_rope
        (OlmoAttention.cpp:111-146), fused

Tensors may be torch tensors on a ROCm device (the call is stream-ordered on
torch's current stream; fp32 selects the exact mode, bf16 the MFMA mode) or
numpy arrays in host memory (copied in, computed and copied out
synchronously, like the reference's value semantics). Everything runs in
libdirktensor_amd.so; nothing here computes attention itself.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

import numpy as np

from . import _capi as C

try:  # torch is plumbing for device memory and streams only
    import torch
except Exception:  # pragma: no cover - torch is installed in every supported environment
    torch = None


class Context:
    """Owns a dt_ctx (device binding, RoPE tables, rocBLAS handle, staging buffers)."""

    def __init__(self, device: int = 0):
        h = ctypes.c_void_p()
        C.call("dt_ctx_create", int(device), ctypes.byref(h))
        self.handle = h
        self.device = int(device)

    def close(self) -> None:
        if self.handle:
            C.lib().dt_ctx_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):  # pragma: no cover - interpreter teardown order
        try:
            self.close()
        except Exception:
            pass

    def rope_table_init(self, theta: float, max_seq_len: int) -> None:
        C.call("dt_rope_table_init", self.handle, float(theta), int(max_seq_len))

    def set_qkv_path(self, path: str) -> None:
        """How layer forwards on this context compute the Q/K/V projection with the q/k norms and RoPE: "fused"
        (one fused kernel), "gemm" (library GEMM, then the norm + RoPE kernel) or "auto" (the default: fused
        where its tiles fit one round on the device's CUs)."""
        values = {"gemm": C.DT_QKV_GEMM, "fused": C.DT_QKV_FUSED, "auto": C.DT_QKV_AUTO}
        if path not in values:
            raise ValueError(f"unknown QKV path {path!r}: expected one of {sorted(values)}")
        C.call("dt_ctx_set_option", self.handle, C.DT_OPT_QKV_FUSED, values[path])

    def set_gemm_tune(self, tune: bool) -> None:
        """bf16 GEMMs of a new shape: time hipBLASLt's heuristic candidates once and keep the fastest reproducible
        one (True, the default), or take its first heuristic choice (False)."""
        C.call("dt_ctx_set_option", self.handle, C.DT_OPT_GEMM_TUNE, int(bool(tune)))

    def set_bwd_dq_path(self, path: str) -> None:
        """How attention backwards on this context form dQ: "recompute" (the dQ pass recomputes S and dP),
        "from_ds" (the dK/dV pass stores dS in a context buffer and dQ = dS K reads it) or "auto" (the default:
        the dS path with more than one 128-row block per CU and pass)."""
        values = {"recompute": C.DT_BWD_DQ_RECOMPUTE, "from_ds": C.DT_BWD_DQ_FROM_DS, "auto": C.DT_BWD_DQ_AUTO}
        if path not in values:
            raise ValueError(f"unknown backward dQ path {path!r}: expected one of {sorted(values)}")
        C.call("dt_ctx_set_option", self.handle, C.DT_OPT_BWD_DQ, values[path])

    def set_qkv_spin_limit(self, polls: int) -> None:
        """Polls a workgroup of the fused QKV kernel waits for the other heads' row sums before it gives up
        (default 2^20, about a second; 0 makes every wait give up, which writes NaN rows and sets the status
        that check() reports)."""
        C.call("dt_ctx_set_option", self.handle, C.DT_OPT_QKV_SPIN_LIMIT, int(polls))

    def set_side_stream(self, on: bool) -> None:
        """Model backwards on this context run their weight-gradient GEMMs and norm-weight column sums on a
        second stream beside the input-gradient chain (True, the default; the same results) or everything on the
        caller's stream (False)."""
        C.call("dt_ctx_set_option", self.handle, C.DT_OPT_SIDE_STREAM, int(bool(on)))

    def check(self) -> None:
        """Waits for the device, then raises DTError (DT_ERR_HIP) when a fused QKV wait gave up since the last
        check."""
        C.call("dt_ctx_check", self.handle)


_default_ctx: dict = {}


def default_context(device: int = 0) -> Context:
    ctx = _default_ctx.get(device)
    if ctx is None:
        ctx = Context(device)
        _default_ctx[device] = ctx
    return ctx


@dataclass
class FlashAttentionResult:
    """FlashAttention.h:6-10: output [B,T,H,D], softmax_m and softmax_l [B,T,H]."""

    output: object
    softmax_m: object
    softmax_l: object


def _is_torch(x) -> bool:
    return torch is not None and isinstance(x, torch.Tensor)


def _mode_of(x, mode: Optional[str]) -> int:
    if mode is not None:
        if mode in ("fp32", "fp32_exact", "exact"):
            return C.DT_FP32_EXACT
        if mode == "bf16":
            return C.DT_BF16
        raise ValueError(f"unknown mode {mode!r}")
    if _is_torch(x):
        if x.dtype == torch.float32:
            return C.DT_FP32_EXACT
        if x.dtype == torch.bfloat16:
            return C.DT_BF16
        raise TypeError(f"unsupported dtype {x.dtype}: use float32 (exact mode) or bfloat16 (MFMA mode)")
    if x.dtype == np.float32:
        return C.DT_FP32_EXACT
    if x.dtype == np.uint16:  # bf16 bit patterns
        return C.DT_BF16
    raise TypeError(f"unsupported numpy dtype {x.dtype}: float32, or uint16 holding bf16 bits")


def _stream_of(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _seq_lens_arg(seq_lens, B: int):
    if seq_lens is None:
        return None, None
    arr = np.ascontiguousarray(np.asarray(seq_lens.cpu() if _is_torch(seq_lens) else seq_lens, dtype=np.int32))
    if arr.shape != (B,):
        raise ValueError(f"seq_lens must have shape ({B},), got {arr.shape}")
    return arr, arr.ctypes.data_as(ctypes.c_void_p)


def flash_attention_forward(Q, K, V, scale: float, causal: bool = True, *, seq_lens=None,
                            mode: Optional[str] = None, ctx: Optional[Context] = None) -> FlashAttentionResult:
    """Causal flash attention forward (FlashAttention.cpp:24-182) on the GPU.

    Q, K, V: [B, T, H, 128], all torch device tensors or all numpy host arrays.
    ``seq_lens`` (optional, B ints in [1, T]) masks keys at t >= seq_lens[b]
    and returns rows t >= seq_lens[b] as the reference's empty row
    (output 0, m = -inf, l = 0). Raises DTError on invalid arguments.
    """
    if Q.shape != K.shape or Q.shape != V.shape or len(Q.shape) != 4:
        raise ValueError(f"Q, K, V must share one [B,T,H,D] shape, got {tuple(Q.shape)}, {tuple(K.shape)}, "
                         f"{tuple(V.shape)}")
    B, T, H, D = (int(s) for s in Q.shape)
    dtype = _mode_of(Q, mode)
    lens_arr, lens_p = _seq_lens_arg(seq_lens, B)
    if _is_torch(Q):
        if not (_is_torch(K) and _is_torch(V)):
            raise TypeError("Q, K, V must all be torch tensors or all numpy arrays")
        if not (Q.is_cuda and K.is_cuda and V.is_cuda):
            raise ValueError("torch inputs must be on a ROCm device; use numpy arrays for host memory")
        if Q.dtype != K.dtype or Q.dtype != V.dtype:
            raise TypeError("Q, K, V must share one dtype")
        ctx = ctx or default_context(Q.device.index or 0)
        Q, K, V = Q.contiguous(), K.contiguous(), V.contiguous()
        O = torch.empty_like(Q)
        m = torch.empty((B, T, H), dtype=torch.float32, device=Q.device)
        l = torch.empty((B, T, H), dtype=torch.float32, device=Q.device)
        C.call("dt_flash_attn_fwd", ctx.handle, Q.data_ptr(), K.data_ptr(), V.data_ptr(), O.data_ptr(),
               m.data_ptr(), l.data_ptr(), B, T, H, D, float(scale), int(bool(causal)), lens_p, dtype,
               C.DT_MEM_DEVICE, _stream_of(Q))
        return FlashAttentionResult(O, m, l)
    ctx = ctx or default_context(0)
    np_dt = np.float32 if dtype == C.DT_FP32_EXACT else np.uint16
    Qh, Kh, Vh = (np.ascontiguousarray(x, dtype=np_dt) for x in (Q, K, V))
    O = np.empty_like(Qh)
    m = np.empty((B, T, H), dtype=np.float32)
    l = np.empty((B, T, H), dtype=np.float32)
    C.call("dt_flash_attn_fwd", ctx.handle, Qh.ctypes.data, Kh.ctypes.data, Vh.ctypes.data, O.ctypes.data,
           m.ctypes.data, l.ctypes.data, B, T, H, D, float(scale), int(bool(causal)), lens_p, dtype,
           C.DT_MEM_HOST, None)
    return FlashAttentionResult(O, m, l)


@dataclass
class FlashAttentionGradients:
    """FlashAttention.h:27-31: d_Q, d_K, d_V [B,T,H,D]."""

    d_Q: object
    d_K: object
    d_V: object


def flash_attention_backward(d_output, output, softmax_m, softmax_l, Q, K, V, scale: float, causal: bool = True, *,
                             mode: Optional[str] = None, ctx: Optional[Context] = None) -> FlashAttentionGradients:
    """Flash attention backward (FlashAttention.cpp:185-359) on the GPU.

    d_output, output, Q, K, V: [B, T, H, 128] in one dtype (fp32: exact mode, bf16: MFMA mode), all torch
    device tensors or all numpy host arrays; softmax_m, softmax_l: the forward's [B, T, H] fp32
    statistics. Returns the three gradients in the inputs' dtype.
    """
    shape = tuple(Q.shape)
    for name, x in (("d_output", d_output), ("output", output), ("K", K), ("V", V)):
        if tuple(x.shape) != shape:
            raise ValueError(f"{name} has shape {tuple(x.shape)}, expected {shape}")
    if len(shape) != 4:
        raise ValueError(f"expected [B,T,H,D] tensors, got {shape}")
    B, T, H, D = shape
    if tuple(softmax_m.shape) != (B, T, H) or tuple(softmax_l.shape) != (B, T, H):
        raise ValueError("softmax_m and softmax_l must have shape [B, T, H]")
    dtype = _mode_of(Q, mode)
    if _is_torch(Q):
        ins = [t.contiguous() for t in (d_output, output, Q, K, V)]
        if any(not _is_torch(t) or not t.is_cuda or t.dtype != Q.dtype for t in ins):
            raise TypeError("d_output, output, Q, K, V must be torch device tensors of one dtype")
        m, l = softmax_m.contiguous().float(), softmax_l.contiguous().float()
        ctx = ctx or default_context(Q.device.index or 0)
        dQ, dK, dV = (torch.empty_like(ins[2]) for _ in range(3))
        C.call("dt_flash_attn_bwd", ctx.handle, ins[0].data_ptr(), ins[1].data_ptr(), m.data_ptr(), l.data_ptr(),
               ins[2].data_ptr(), ins[3].data_ptr(), ins[4].data_ptr(), dQ.data_ptr(), dK.data_ptr(), dV.data_ptr(),
               B, T, H, D, float(scale), int(bool(causal)), dtype, C.DT_MEM_DEVICE, _stream_of(Q))
        return FlashAttentionGradients(dQ, dK, dV)
    ctx = ctx or default_context(0)
    np_dt = np.float32 if dtype == C.DT_FP32_EXACT else np.uint16
    ins = [np.ascontiguousarray(x, dtype=np_dt) for x in (d_output, output, Q, K, V)]
    m = np.ascontiguousarray(softmax_m, dtype=np.float32)
    l = np.ascontiguousarray(softmax_l, dtype=np.float32)
    dQ, dK, dV = (np.empty_like(ins[2]) for _ in range(3))
    C.call("dt_flash_attn_bwd", ctx.handle, ins[0].ctypes.data, ins[1].ctypes.data, m.ctypes.data, l.ctypes.data,
           ins[2].ctypes.data, ins[3].ctypes.data, ins[4].ctypes.data, dQ.ctypes.data, dK.ctypes.data,
           dV.ctypes.data, B, T, H, D, float(scale), int(bool(causal)), dtype, C.DT_MEM_HOST, None)
    return FlashAttentionGradients(dQ, dK, dV)


def qk_norm_rope(q_proj, k_proj, q_norm_w, k_norm_w, *, n_heads: int = C.N_HEADS, out_dtype: str = "fp32",
                 return_rms: bool = False, ctx: Optional[Context] = None):
    """Fused q/k RMSNorm over all d_model features + rotate-half RoPE at position t.

    q_proj, k_proj: [B, T, d_model] fp32; returns q, k as [B, T, H, 128]
    (fp32, or bf16 when out_dtype == "bf16"), plus the two [B, T] rms arrays
    when ``return_rms``.
    """
    B, T, dm = (int(s) for s in q_proj.shape)
    H = n_heads
    od = C.DT_BF16 if out_dtype == "bf16" else C.DT_FP32_EXACT
    if _is_torch(q_proj):
        ctx = ctx or default_context(q_proj.device.index or 0)
        q_in, k_in = q_proj.contiguous(), k_proj.contiguous()
        tdt = torch.bfloat16 if od == C.DT_BF16 else torch.float32
        q_out = torch.empty((B, T, H, dm // H), dtype=tdt, device=q_in.device)
        k_out = torch.empty_like(q_out)
        q_rms = torch.empty((B, T), dtype=torch.float32, device=q_in.device)
        k_rms = torch.empty_like(q_rms)
        C.call("dt_qk_norm_rope_fwd", ctx.handle, q_in.data_ptr(), k_in.data_ptr(), q_norm_w.contiguous().data_ptr(),
               k_norm_w.contiguous().data_ptr(), q_out.data_ptr(), k_out.data_ptr(), q_rms.data_ptr(),
               k_rms.data_ptr(), B, T, H, dm // H, dm, dm, od, C.DT_MEM_DEVICE, _stream_of(q_in))
    else:
        ctx = ctx or default_context(0)
        q_in = np.ascontiguousarray(q_proj, dtype=np.float32)
        k_in = np.ascontiguousarray(k_proj, dtype=np.float32)
        qw = np.ascontiguousarray(q_norm_w, dtype=np.float32)
        kw = np.ascontiguousarray(k_norm_w, dtype=np.float32)
        ndt = np.uint16 if od == C.DT_BF16 else np.float32
        q_out = np.empty((B, T, H, dm // H), dtype=ndt)
        k_out = np.empty_like(q_out)
        q_rms = np.empty((B, T), dtype=np.float32)
        k_rms = np.empty_like(q_rms)
        C.call("dt_qk_norm_rope_fwd", ctx.handle, q_in.ctypes.data, k_in.ctypes.data, qw.ctypes.data,
               kw.ctypes.data, q_out.ctypes.data, k_out.ctypes.data, q_rms.ctypes.data, k_rms.ctypes.data,
               B, T, H, dm // H, dm, dm, od, C.DT_MEM_HOST, None)
    if return_rms:
        return q_out, k_out, q_rms, k_rms
    return q_out, k_out


class OlmoAttention:
    """OlmoAttention (OlmoAttention.h:10-42) on the HIP path.

    ``OlmoAttention(folder, index)`` loads the reference's per-layer .npy files
    (OlmoAttention.cpp:39-53); ``OlmoAttention.from_weights`` takes arrays
    (fp32, [out, in] like torch Linear). ``forward(x)`` maps [B, T, d_model]
    fp32 to [B, T, d_model] fp32 (OlmoAttention.cpp:56-108); backward, step and
    zero_grad follow OlmoAttention.cpp:193-330.
    """

    def __init__(self, folder: Optional[str] = None, index: int = 0, *, ctx: Optional[Context] = None,
                 _handle: Optional[ctypes.c_void_p] = None):
        self.ctx = ctx or default_context(0)
        self.d_model = None
        if _handle is not None:
            self.handle = _handle
            return
        if folder is None:
            raise ValueError("OlmoAttention needs a weights folder (or use OlmoAttention.from_weights)")
        h = ctypes.c_void_p()
        C.call("dt_attn_layer_load", self.ctx.handle, str(folder).encode(), int(index), ctypes.byref(h))
        self.handle = h
        self.d_model = int(np.load(f"{folder}/model.layers.{index}.self_attn.q_norm.weight.npy",
                                   mmap_mode="r").shape[0])

    @classmethod
    def from_weights(cls, wq, wk, wv, wo, q_norm, k_norm, *, ctx: Optional[Context] = None) -> "OlmoAttention":
        ctx = ctx or default_context(0)
        dm = int(wq.shape[0])
        h = ctypes.c_void_p()
        if _is_torch(wq):
            ws = [w.contiguous().float() for w in (wq, wk, wv, wo, q_norm, k_norm)]
            C.call("dt_attn_layer_create", ctx.handle, *[w.data_ptr() for w in ws], dm, dm // C.HEAD_DIM,
                   C.DT_MEM_DEVICE, ctypes.byref(h))
            torch.cuda.synchronize(ws[0].device)
        else:
            ws = [np.ascontiguousarray(w, dtype=np.float32) for w in (wq, wk, wv, wo, q_norm, k_norm)]
            C.call("dt_attn_layer_create", ctx.handle, *[w.ctypes.data for w in ws], dm, dm // C.HEAD_DIM,
                   C.DT_MEM_HOST, ctypes.byref(h))
        layer = cls(ctx=ctx, _handle=h)
        layer.d_model = dm
        return layer

    def close(self) -> None:
        if getattr(self, "handle", None):
            C.lib().dt_attn_layer_destroy(self.handle)
            self.handle = None

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass

    def forward(self, x, *, seq_lens=None, mode: str = "fp32", save_for_backward: Optional[bool] = None):
        """OlmoAttention::forward. Keeps the state backward needs (as the reference always does) unless
        ``save_for_backward`` is False; the default keeps it for full sequences and not with ``seq_lens``
        (the backward covers full sequences only)."""
        B, T, dm = (int(s) for s in x.shape)
        dtype = _mode_of(x, mode)
        lens_arr, lens_p = _seq_lens_arg(seq_lens, B)
        save = int(seq_lens is None) if save_for_backward is None else int(bool(save_for_backward))
        if _is_torch(x):
            xi = x.contiguous().float()
            out = torch.empty_like(xi)
            C.call("dt_attn_layer_fwd", self.handle, xi.data_ptr(), out.data_ptr(), B, T, lens_p, dtype,
                   C.DT_MEM_DEVICE, save, _stream_of(xi))
            return out
        xi = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty_like(xi)
        C.call("dt_attn_layer_fwd", self.handle, xi.ctypes.data, out.ctypes.data, B, T, lens_p, dtype,
               C.DT_MEM_HOST, save, None)
        return out

    __call__ = forward

    def backward(self, d_output):
        """OlmoAttention::backward (OlmoAttention.cpp:193-312): returns d_input and accumulates the
        parameter gradients, for the last forward that kept its state."""
        B, T, dm = (int(s) for s in d_output.shape)
        if _is_torch(d_output):
            g = d_output.contiguous().float()
            dx = torch.empty_like(g)
            C.call("dt_attn_layer_bwd", self.handle, g.data_ptr(), dx.data_ptr(), B, T, C.DT_MEM_DEVICE,
                   _stream_of(g))
            return dx
        g = np.ascontiguousarray(d_output, dtype=np.float32)
        dx = np.empty_like(g)
        C.call("dt_attn_layer_bwd", self.handle, g.ctypes.data, dx.ctypes.data, B, T, C.DT_MEM_HOST, None)
        return dx

    def step(self, lr: float):
        """OlmoAttention::step (OlmoAttention.cpp:314-321): w -= lr * grad."""
        C.call("dt_attn_layer_step", self.handle, float(lr), self._stream())

    def zero_grad(self):
        """OlmoAttention::zero_grad (OlmoAttention.cpp:323-330)."""
        C.call("dt_attn_layer_zero_grad", self.handle, self._stream())

    def _stream(self):
        if torch is not None and torch.cuda.is_available():
            return ctypes.c_void_p(torch.cuda.current_stream(self.ctx.device).cuda_stream)
        return None

    def _copy_out(self, fn: str) -> dict:
        dm = self._d_model()
        arrs = {k: np.empty((dm, dm), np.float32) for k in ("wq", "wk", "wv", "wo")}
        arrs["q_norm"] = np.empty(dm, np.float32)
        arrs["k_norm"] = np.empty(dm, np.float32)
        C.call(fn, self.handle, *[arrs[k].ctypes.data for k in ("wq", "wk", "wv", "wo", "q_norm", "k_norm")],
               C.DT_MEM_HOST, self._stream())
        return arrs

    def _d_model(self) -> int:
        if getattr(self, "d_model", None) is None:
            raise RuntimeError("d_model unknown: construct with from_weights or pass d_model")
        return self.d_model

    def weights(self) -> dict:
        """Host copies of Wq, Wk, Wv, Wo, q_norm, k_norm (the param<2>::w members)."""
        return self._copy_out("dt_attn_layer_get_weights")

    def grads(self) -> dict:
        """Host copies of the accumulated gradients (the param<2>::grad members)."""
        return self._copy_out("dt_attn_layer_get_grads")
