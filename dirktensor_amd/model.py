"""Python mirror of the reference's OlmoModel (OlmoModel.h:14-34) and ce_loss (CrossEntropyLoss.h:10-13)
on the HIP path: every method calls libdirktensor_amd.so; nothing here computes the model.

    OlmoModel(folder, n_layers=16)            OlmoModel.cpp:12-23 (reads the .npy files)
    OlmoModel.from_params(params)             seeded / caller-provided weights keyed by file stem
    forward(batch) -> logits                  OlmoModel.cpp:25-48
    backward(d_logits), step(lr), zero_grad() OlmoModel.cpp:50-83
    ce_loss(logits, batch, ignore_index)      CrossEntropyLoss.cpp:8-43 (+ main.cpp:62-80's gradient)
"""

from __future__ import annotations

import ctypes
import re
from typing import Optional

import numpy as np

from . import _capi as C
from .attention import Context, _is_torch, _mode_of, _stream_of, default_context, torch

PAD_TOKEN = 100277  # <|pad|> (vocab.txt:100278, Detokenizer.cpp:76-77)


class OlmoModel:
    def __init__(self, folder: Optional[str] = None, n_layers: int = 16, *, ctx: Optional[Context] = None,
                 _handle=None, _dims=None):
        self.ctx = ctx or default_context(0)
        if _handle is not None:
            self.handle = _handle
            self.n_layers, self.d_model, self.hidden, self.vocab = _dims
            return
        if folder is None:
            raise ValueError("OlmoModel needs a weights folder (or use OlmoModel.from_params)")
        h = ctypes.c_void_p()
        C.call("dt_model_load", self.ctx.handle, str(folder).encode(), int(n_layers), ctypes.byref(h))
        self.handle = h
        emb = np.load(f"{folder}/model.embed_tokens.weight.npy", mmap_mode="r")
        up = np.load(f"{folder}/model.layers.0.mlp.up_proj.weight.npy", mmap_mode="r")
        self.n_layers, self.d_model, self.hidden, self.vocab = n_layers, emb.shape[1], up.shape[0], emb.shape[0]

    @classmethod
    def from_params(cls, params: dict, *, ctx: Optional[Context] = None) -> "OlmoModel":
        ctx = ctx or default_context(0)
        V, dm = params["model.embed_tokens.weight"].shape
        hid = params["model.layers.0.mlp.up_proj.weight"].shape[0]
        n_layers = 1 + max(int(m.group(1)) for k in params if (m := re.match(r"model\.layers\.(\d+)\.", k)))
        h = ctypes.c_void_p()
        C.call("dt_model_create", ctx.handle, n_layers, dm, dm // C.HEAD_DIM, hid, V, ctypes.byref(h))
        model = cls(ctx=ctx, _handle=h, _dims=(n_layers, dm, hid, V))
        for name, arr in params.items():
            model.set_param(name, arr)
        return model

    def close(self) -> None:
        if getattr(self, "handle", None):
            C.lib().dt_model_destroy(self.handle)
            self.handle = None

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass

    def _stream(self):
        if torch is not None and torch.cuda.is_available():
            return ctypes.c_void_p(torch.cuda.current_stream(self.ctx.device).cuda_stream)
        return None

    def set_param(self, name: str, arr) -> None:
        a = np.ascontiguousarray(arr, dtype=np.float32)
        C.call("dt_model_set_param", self.handle, name.encode(), a.ctypes.data, a.size, C.DT_MEM_HOST)

    def _shape(self, name: str):
        dm, hid, V = self.d_model, self.hidden, self.vocab
        if name in ("model.embed_tokens.weight", "lm_head.weight"):
            return (V, dm)
        if name.endswith(("norm.weight", "layernorm.weight")):
            return (dm,)
        if name.endswith(("gate_proj.weight", "up_proj.weight")):
            return (hid, dm)
        if name.endswith("down_proj.weight"):
            return (dm, hid)
        return (dm, dm)

    def param(self, name: str, grad: bool = False) -> np.ndarray:
        out = np.empty(self._shape(name), np.float32)
        C.call("dt_model_get_param", self.handle, name.encode(), out.ctypes.data, out.size, int(grad), C.DT_MEM_HOST,
               self._stream())
        return out

    def grad(self, name: str) -> np.ndarray:
        return self.param(name, grad=True)

    def forward(self, batch, *, mode: str = "fp32", save_for_backward: bool = True, out=None):
        """OlmoModel::forward: batch [B, T] token ids (host array) -> logits [B, T, vocab] fp32 (a device tensor
        when ``out`` is one, else a numpy array)."""
        tok = np.ascontiguousarray(batch.cpu().numpy() if _is_torch(batch) else batch, dtype=np.int32)
        B, T = tok.shape
        dtype = _mode_of(np.zeros(1, np.float32), mode)
        if out is not None and _is_torch(out):
            C.call("dt_model_fwd", self.handle, tok.ctypes.data, B, T, out.data_ptr(), dtype, C.DT_MEM_DEVICE,
                   int(bool(save_for_backward)), _stream_of(out))
            return out
        logits = np.empty((B, T, self.vocab), np.float32)
        C.call("dt_model_fwd", self.handle, tok.ctypes.data, B, T, logits.ctypes.data, dtype, C.DT_MEM_HOST,
               int(bool(save_for_backward)), None)
        return logits

    __call__ = forward

    def backward(self, d_logits) -> None:
        if _is_torch(d_logits):
            g = d_logits.contiguous().float()
            C.call("dt_model_bwd", self.handle, g.data_ptr(), C.DT_MEM_DEVICE, _stream_of(g))
        else:
            g = np.ascontiguousarray(d_logits, dtype=np.float32)
            C.call("dt_model_bwd", self.handle, g.ctypes.data, C.DT_MEM_HOST, None)

    def step(self, lr: float) -> None:
        C.call("dt_model_step", self.handle, float(lr), self._stream())

    def zero_grad(self) -> None:
        C.call("dt_model_zero_grad", self.handle, self._stream())


def ce_loss(logits, batch, ignore_index: int = PAD_TOKEN, *, with_grad: bool = False, ctx: Optional[Context] = None):
    """ce_loss (CrossEntropyLoss.cpp:8-43) on the GPU: the mean next-token cross entropy, targets equal to
    ``ignore_index`` skipped. With ``with_grad`` also returns main.cpp:62-80's gradient w.r.t. the logits."""
    tok = np.ascontiguousarray(batch.cpu().numpy() if _is_torch(batch) else batch, dtype=np.int32)
    B, T, V = (int(s) for s in logits.shape)
    loss = np.zeros(1, np.float32)
    if _is_torch(logits):
        ctx = ctx or default_context(logits.device.index or 0)
        lg = logits.contiguous().float()
        g = torch.empty_like(lg) if with_grad else None
        C.call("dt_ce_loss", ctx.handle, lg.data_ptr(), tok.ctypes.data, B, T, V, int(ignore_index), loss.ctypes.data,
               g.data_ptr() if g is not None else None, C.DT_MEM_DEVICE, _stream_of(lg))
    else:
        ctx = ctx or default_context(0)
        lg = np.ascontiguousarray(logits, dtype=np.float32)
        g = np.empty_like(lg) if with_grad else None
        C.call("dt_ce_loss", ctx.handle, lg.ctypes.data, tok.ctypes.data, B, T, V, int(ignore_index), loss.ctypes.data,
               g.ctypes.data if g is not None else None, C.DT_MEM_HOST, None)
    return (float(loss[0]), g) if with_grad else float(loss[0])
