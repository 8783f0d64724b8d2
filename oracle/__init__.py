"""CPU oracle for the attention path — TEST INFRASTRUCTURE ONLY.

ctypes wrapper of oracle/liboracle.so (built from oracle/dt_oracle.cpp by
oracle/Makefile). Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use it, to verify the GPU results or as the timed CPU
baseline; the product path (dirktensor_amd) never imports it.

Each function names the reference code it restates; see dt_oracle.cpp.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
_lib = None

_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float


def build() -> Path:
    subprocess.run(["make", "-B", "-s", "-C", os.fspath(HERE)], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        l = ctypes.CDLL(os.fspath(LIB_PATH))
        l.oracle_version.restype = _i
        l.oracle_set_mutation.argtypes = [_i]
        l.oracle_get_mutation.restype = _i
        l.oracle_rope_tables.argtypes = [_vp, _vp, _i, _i, _f]
        l.oracle_apply_rope.argtypes = [_vp, _vp, _i, _i, _i, _i, _vp, _vp]
        l.oracle_rmsnorm_forward.argtypes = [_vp, _vp, _vp, _vp, _i, _i, _f]
        l.oracle_flash_attention_forward.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _f, _i, _i]
        l.oracle_sgemm_nt.argtypes = [_i, _i, _i, _f, _vp, _i, _vp, _i, _vp, _i, _i]
        l.oracle_attention_layer_forward.argtypes = [_vp] * 9 + [_vp, _i, _i, _i, _i, _f, _i] + [_vp] * 6
        l.oracle_flash_attention_backward.argtypes = [_vp] * 10 + [_i, _i, _i, _i, _f, _i, _i]
        l.oracle_apply_rope_backward.argtypes = [_vp, _vp, _i, _i, _i, _i, _vp, _vp]
        l.oracle_rmsnorm_backward.argtypes = [_vp] * 6 + [_i, _i]
        l.oracle_attention_layer_backward.argtypes = [_vp] * 17 + [_i, _i, _i, _i, _f, _i]
        l.oracle_mlp_forward.argtypes = [_vp] * 5 + [_i, _i, _i, _i, _vp, _vp, _vp]
        l.oracle_model_forward.argtypes = [_vp] * 6 + [_i] * 6 + [_f, _i]
        l.oracle_ce_loss.argtypes = [_vp, _vp, _i, _i, _i, _i, _vp, _vp]
        l.oracle_ce_loss.restype = _f
        l.oracle_model_backward.argtypes = [_vp] * 10 + [_i] * 6 + [_f, _i]
        _lib = l
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(_vp)


def _c32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def default_threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


class mutation:
    """Context manager planting a known mistake in the oracle (tests only)."""

    def __init__(self, m: int):
        self.m = m

    def __enter__(self):
        lib().oracle_set_mutation(self.m)

    def __exit__(self, *exc):
        lib().oracle_set_mutation(0)


def rope_tables(max_seq: int = 8192, D: int = 128, theta: float = 500000.0):
    """compute_rope_buffers (OlmoAttention.cpp:18-31): sin, cos [max_seq, D] fp32."""
    s = np.empty((max_seq, D), dtype=np.float32)
    c = np.empty((max_seq, D), dtype=np.float32)
    lib().oracle_rope_tables(_p(s), _p(c), max_seq, D, float(theta))
    return s, c


def apply_rope(x, sin_t, cos_t):
    """OlmoAttention::apply_rope (OlmoAttention.cpp:111-146); x [B,T,H,D]."""
    x = _c32(x)
    B, T, H, D = x.shape
    out = np.empty_like(x)
    lib().oracle_apply_rope(_p(x), _p(out), B, T, H, D, _p(_c32(sin_t)), _p(_c32(cos_t)))
    return out


def rmsnorm_forward(x, w, eps: float = 1e-6):
    """RMSNorm::forward (RMSNorm.cpp:15-22) over the last axis; returns (y, rms)."""
    x = _c32(x)
    C = x.shape[-1]
    rows = x.size // C
    y = np.empty_like(x)
    rms = np.empty(x.shape[:-1], dtype=np.float32)
    lib().oracle_rmsnorm_forward(_p(x), _p(_c32(w)), _p(y), _p(rms), rows, C, float(eps))
    return y, rms


def flash_attention_forward(Q, K, V, scale: float, causal: bool = True, nthreads: int | None = None):
    """flash_attention_forward (FlashAttention.cpp:24-182); returns (O, m, l)."""
    Q, K, V = _c32(Q), _c32(K), _c32(V)
    B, T, H, D = Q.shape
    O = np.empty_like(Q)
    m = np.empty((B, T, H), dtype=np.float32)
    l = np.empty((B, T, H), dtype=np.float32)
    lib().oracle_flash_attention_forward(_p(Q), _p(K), _p(V), _p(O), _p(m), _p(l), B, T, H, D, float(scale),
                                         int(bool(causal)), nthreads or default_threads())
    return O, m, l


def flash_attention_ragged(Q, K, V, seq_lens, scale: float, nthreads: int | None = None):
    """Reference semantics of a right-padded batch: each sequence b run alone on its
    unpadded prefix [0, L_b) (causal rows t < L_b never see later keys); rows t >= L_b
    get the reference's empty row (O = 0, m = -inf, l = 0, FlashAttention.cpp:165-174)."""
    Q, K, V = _c32(Q), _c32(K), _c32(V)
    B, T, H, D = Q.shape
    O = np.zeros_like(Q)
    m = np.full((B, T, H), -np.inf, dtype=np.float32)
    l = np.zeros((B, T, H), dtype=np.float32)
    for b in range(B):
        L = int(seq_lens[b])
        o, mm, ll = flash_attention_forward(Q[b:b + 1, :L], K[b:b + 1, :L], V[b:b + 1, :L], scale, True, nthreads)
        O[b, :L], m[b, :L], l[b, :L] = o[0], mm[0], ll[0]
    return O, m, l


def sgemm_nt(A, B, alpha: float = 1.0, nthreads: int | None = None):
    """C = alpha * A B^T (row-major), the oracle's stand-in for cblas_sgemm(NoTrans, Trans)."""
    A, B = _c32(A), _c32(B)
    M, K = A.shape
    N = B.shape[0]
    Cm = np.empty((M, N), dtype=np.float32)
    lib().oracle_sgemm_nt(M, N, K, float(alpha), _p(A), K, _p(B), K, _p(Cm), N, nthreads or default_threads())
    return Cm


def attention_layer_forward(x, wq, wk, wv, wo, q_norm, k_norm, *, theta: float = 500000.0, eps: float = 1e-6,
                            nthreads: int | None = None, return_state: bool = False):
    """OlmoAttention::forward (OlmoAttention.cpp:56-108) for x [B,T,d_model]."""
    x = _c32(x)
    B, T, dm = x.shape
    D = 128
    H = dm // D
    sin_t, cos_t = rope_tables(max(T, 1), D, theta)
    out = np.empty_like(x)
    st = None
    if return_state:
        st = dict(q_rope=np.empty((B, T, H, D), np.float32), k_rope=np.empty((B, T, H, D), np.float32),
                  v=np.empty((B, T, H, D), np.float32), attn=np.empty((B, T, H, D), np.float32),
                  m=np.empty((B, T, H), np.float32), l=np.empty((B, T, H), np.float32))
    g = (lambda k: _p(st[k])) if st else (lambda k: None)
    lib().oracle_attention_layer_forward(_p(x), _p(_c32(wq)), _p(_c32(wk)), _p(_c32(wv)), _p(_c32(wo)),
                                         _p(_c32(q_norm)), _p(_c32(k_norm)), _p(sin_t), _p(cos_t), _p(out),
                                         B, T, H, D, float(eps), nthreads or default_threads(),
                                         g("q_rope"), g("k_rope"), g("v"), g("attn"), g("m"), g("l"))
    return (out, st) if return_state else out


def flash_attention_backward(dO, O, m, l, Q, K, V, scale: float, causal: bool = True, nthreads: int | None = None):
    """flash_attention_backward (FlashAttention.cpp:185-359); returns (dQ, dK, dV)."""
    dO, O, m, l, Q, K, V = (_c32(a) for a in (dO, O, m, l, Q, K, V))
    B, T, H, D = Q.shape
    dQ, dK, dV = np.empty_like(Q), np.empty_like(Q), np.empty_like(Q)
    lib().oracle_flash_attention_backward(_p(dO), _p(O), _p(m), _p(l), _p(Q), _p(K), _p(V), _p(dQ), _p(dK), _p(dV),
                                          B, T, H, D, float(scale), int(bool(causal)), nthreads or default_threads())
    return dQ, dK, dV


def apply_rope_backward(d_out, sin_t, cos_t):
    """OlmoAttention::apply_rope_backward (OlmoAttention.cpp:149-190); d_out [B,T,H,D]."""
    d_out = _c32(d_out)
    B, T, H, D = d_out.shape
    d_in = np.empty_like(d_out)
    lib().oracle_apply_rope_backward(_p(d_out), _p(d_in), B, T, H, D, _p(_c32(sin_t)), _p(_c32(cos_t)))
    return d_in


def rmsnorm_backward(dy, y, rms, w):
    """RMSNorm::backward (RMSNorm.cpp:24-36) from the forward's output y and rms; returns (dx, dw)."""
    dy, y, rms, w = _c32(dy), _c32(y), _c32(rms), _c32(w)
    C = y.shape[-1]
    rows = y.size // C
    dx = np.empty_like(y)
    dw = np.zeros(C, dtype=np.float32)
    lib().oracle_rmsnorm_backward(_p(dy), _p(y), _p(rms), _p(w), _p(dx), _p(dw), rows, C)
    return dx, dw


def attention_layer_backward(x, wq, wk, wv, wo, q_norm, k_norm, d_out, *, theta: float = 500000.0,
                             eps: float = 1e-6, nthreads: int | None = None):
    """OlmoAttention::backward (OlmoAttention.cpp:193-312) after a forward on x [B,T,d_model].
    Returns d_x and the gradients {wq, wk, wv, wo, q_norm, k_norm} accumulated from zero."""
    x, d_out = _c32(x), _c32(d_out)
    B, T, dm = x.shape
    D = 128
    H = dm // D
    sin_t, cos_t = rope_tables(max(T, 1), D, theta)
    d_x = np.empty_like(x)
    g = {k: np.zeros((dm, dm), np.float32) for k in ("wq", "wk", "wv", "wo")}
    g["q_norm"] = np.zeros(dm, np.float32)
    g["k_norm"] = np.zeros(dm, np.float32)
    lib().oracle_attention_layer_backward(_p(x), _p(_c32(wq)), _p(_c32(wk)), _p(_c32(wv)), _p(_c32(wo)),
                                          _p(_c32(q_norm)), _p(_c32(k_norm)), _p(sin_t), _p(cos_t), _p(d_out),
                                          _p(d_x), _p(g["wq"]), _p(g["wk"]), _p(g["wv"]), _p(g["wo"]),
                                          _p(g["q_norm"]), _p(g["k_norm"]), B, T, H, D, float(eps),
                                          nthreads or default_threads())
    return d_x, g


LAYER_PARAMS = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj", "self_attn.q_norm",
                "self_attn.k_norm", "post_attention_layernorm", "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj",
                "post_feedforward_layernorm")


def mlp_forward(x, w_gate, w_up, w_down, nthreads: int | None = None):
    """OlmoMlp::forward (OlmoMlp.cpp:26-63) on rows of x [..., dm]."""
    x = _c32(x)
    dm = x.shape[-1]
    rows = x.size // dm
    hid = w_up.shape[0]
    out = np.empty(x.shape, np.float32)
    lib().oracle_mlp_forward(_p(x), _p(_c32(w_gate)), _p(_c32(w_up)), _p(_c32(w_down)), _p(out), rows, dm, hid,
                             nthreads or default_threads(), None, None, None)
    return out


def model_forward(tokens, params: dict, *, eps: float = 1e-6, nthreads: int | None = None):
    """OlmoModel::forward (OlmoModel.cpp:25-48): tokens [B, T] -> logits [B, T, V]. ``params`` maps the
    reference's weight file stems ("model.embed_tokens.weight", "model.layers.{i}.mlp.up_proj.weight",
    ..., "model.norm.weight", "lm_head.weight") to fp32 arrays."""
    tok = np.ascontiguousarray(tokens, dtype=np.int32)
    B, T = tok.shape
    embed = _c32(params["model.embed_tokens.weight"])
    V, dm = embed.shape
    n_layers = sum(1 for k in params if k.endswith(".mlp.up_proj.weight"))
    hid = params["model.layers.0.mlp.up_proj.weight"].shape[0]
    keep = [embed]
    ptrs = (_vp * (n_layers * len(LAYER_PARAMS)))()
    for i in range(n_layers):
        for j, name in enumerate(LAYER_PARAMS):
            a = _c32(params[f"model.layers.{i}.{name}.weight"])
            keep.append(a)
            ptrs[i * len(LAYER_PARAMS) + j] = a.ctypes.data
    fn, lm = _c32(params["model.norm.weight"]), _c32(params["lm_head.weight"])
    logits = np.empty((B, T, V), np.float32)
    lib().oracle_model_forward(_p(tok), _p(embed), ctypes.cast(ptrs, _vp), _p(fn), _p(lm), _p(logits), B, T, dm, hid,
                               V, n_layers, float(eps), nthreads or default_threads())
    return logits


def ce_loss(logits, tokens, ignore_index: int, with_grad: bool = False):
    """ce_loss (CrossEntropyLoss.cpp:8-43): mean next-token cross entropy, targets tokens[:, 1:], those equal
    to ignore_index skipped. With ``with_grad`` also main.cpp:62-80's gradient (softmax - onehot) / count."""
    logits = _c32(logits)
    tok = np.ascontiguousarray(tokens, dtype=np.int32)
    B, T, V = logits.shape
    g = np.empty_like(logits) if with_grad else None
    cnt = ctypes.c_int(0)
    loss = lib().oracle_ce_loss(_p(logits), _p(tok), B, T, V, int(ignore_index), _p(g), ctypes.byref(cnt))
    return (float(loss), g) if with_grad else float(loss)


def _layer_ptrs(arrays: dict, n_layers: int):
    ptrs = (_vp * (n_layers * len(LAYER_PARAMS)))()
    for i in range(n_layers):
        for j, name in enumerate(LAYER_PARAMS):
            ptrs[i * len(LAYER_PARAMS) + j] = arrays[f"model.layers.{i}.{name}.weight"].ctypes.data
    return ptrs


def model_backward(tokens, params: dict, d_logits, *, eps: float = 1e-6, nthreads: int | None = None) -> dict:
    """OlmoModel::backward (OlmoModel.cpp:50-67) after a forward on ``tokens``: the gradient of every parameter
    (accumulated from zero), keyed like ``params``."""
    tok = np.ascontiguousarray(tokens, dtype=np.int32)
    B, T = tok.shape
    p = {k: _c32(v) for k, v in params.items()}
    V, dm = p["model.embed_tokens.weight"].shape
    n_layers = sum(1 for k in p if k.endswith(".mlp.up_proj.weight"))
    hid = p["model.layers.0.mlp.up_proj.weight"].shape[0]
    g = {k: np.zeros_like(v) for k, v in p.items()}
    dl = _c32(d_logits)
    lib().oracle_model_backward(_p(tok), _p(p["model.embed_tokens.weight"]), ctypes.cast(_layer_ptrs(p, n_layers), _vp),
                                _p(p["model.norm.weight"]), _p(p["lm_head.weight"]), _p(dl),
                                _p(g["model.embed_tokens.weight"]), ctypes.cast(_layer_ptrs(g, n_layers), _vp),
                                _p(g["model.norm.weight"]), _p(g["lm_head.weight"]), B, T, dm, hid, V, n_layers,
                                float(eps), nthreads or default_threads())
    return g
