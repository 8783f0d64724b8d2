"""The C ABI on a host without a GPU: the library loads, exports every declared
symbol, and rejects invalid arguments before its first HIP call."""

import ctypes
import os
import re
import subprocess
import sys

import numpy as np
import pytest

from dirktensor_amd import _capi as C

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dirktensor_amd.h")
FAKE = 0x10000  # aligned non-NULL address; never dereferenced because validation fails first


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dt_[a-z0-9_]+)\s*\(", text)))


def last_error():
    return C.lib().dt_last_error().decode()


def test_every_declared_symbol_is_exported_and_bound():
    names = declared_functions()
    assert len(names) >= 12
    lib = C.lib()
    for n in names:
        assert hasattr(lib, n), f"{n} declared in the header but not exported"
    assert sorted(C.SIGNATURES) == names, "ctypes signature table and header disagree"
    assert lib.dt_version() == 3


def flash(**kw):
    a = dict(ctx=None, q=FAKE, k=FAKE, v=FAKE, o=FAKE, m=None, l=None, B=1, T=64, H=16, D=128, scale=0.088,
             causal=1, seq_lens=None, dtype=C.DT_BF16, mem=C.DT_MEM_DEVICE, stream=None)
    a.update(kw)
    return C.lib().dt_flash_attn_fwd(*a.values())


@pytest.mark.parametrize("kw,code,msg", [
    (dict(D=64), C.DT_ERR_UNSUPPORTED, "head_dim"),
    (dict(T=8193), C.DT_ERR_INVALID_ARG, "max_seq_len"),
    (dict(T=0), C.DT_ERR_INVALID_ARG, ">= 1"),
    (dict(B=0), C.DT_ERR_INVALID_ARG, ">= 1"),
    (dict(q=None), C.DT_ERR_INVALID_ARG, "non-NULL"),
    (dict(dtype=7), C.DT_ERR_INVALID_ARG, "dtype"),
    (dict(mem=5), C.DT_ERR_INVALID_ARG, "mem"),
    (dict(scale=0.0), C.DT_ERR_INVALID_ARG, "scale"),
    (dict(scale=float("nan")), C.DT_ERR_INVALID_ARG, "scale"),
    (dict(causal=2), C.DT_ERR_INVALID_ARG, "causal"),
    (dict(o=FAKE + 4), C.DT_ERR_INVALID_ARG, "aligned"),
    ({}, C.DT_ERR_INVALID_ARG, "ctx is NULL"),
])
def test_flash_validation_before_any_hip_call(kw, code, msg):
    assert flash(**kw) == code
    assert msg in last_error()


def test_flash_seq_lens_validation():
    lens = (ctypes.c_int32 * 2)(64, 65)
    assert flash(B=2, T=64, seq_lens=ctypes.cast(lens, ctypes.c_void_p)) == C.DT_ERR_INVALID_ARG
    assert "seq_lens[1]=65" in last_error()
    lens0 = (ctypes.c_int32 * 1)(0)
    assert flash(B=1, seq_lens=ctypes.cast(lens0, ctypes.c_void_p)) == C.DT_ERR_INVALID_ARG
    big = (ctypes.c_int32 * 300)(*([1] * 300))
    assert flash(B=300, seq_lens=ctypes.cast(big, ctypes.c_void_p)) == C.DT_ERR_UNSUPPORTED


def test_flash_bwd_validation():
    """dt_flash_attn_bwd rejects bad arguments before any HIP call (no device is touched here)."""
    lib = C.lib()
    args = [None] + [FAKE] * 10 + [1, 64, 2, 128, 0.1, 1, C.DT_BF16, C.DT_MEM_DEVICE, None]
    assert lib.dt_flash_attn_bwd(*args) == C.DT_ERR_INVALID_ARG and "ctx is NULL" in last_error()
    bad = list(args)
    bad[3] = None  # l
    assert lib.dt_flash_attn_bwd(*bad) == C.DT_ERR_INVALID_ARG and "non-NULL" in last_error()
    bad = list(args)
    bad[14] = 96
    assert lib.dt_flash_attn_bwd(*bad) == C.DT_ERR_UNSUPPORTED
    bad = list(args)
    bad[12] = 9000
    assert lib.dt_flash_attn_bwd(*bad) == C.DT_ERR_INVALID_ARG
    bad = list(args)
    bad[17] = 7
    assert lib.dt_flash_attn_bwd(*bad) == C.DT_ERR_INVALID_ARG and "dtype" in last_error()
    bad = list(args)
    bad[15] = -1.0
    assert lib.dt_flash_attn_bwd(*bad) == C.DT_ERR_INVALID_ARG and "scale" in last_error()


def test_norm_rope_and_layer_validation():
    lib = C.lib()
    args = [None, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None, None, 1, 16, 16, 128, 2048, 2048, C.DT_FP32_EXACT,
            C.DT_MEM_DEVICE, None]
    assert lib.dt_qk_norm_rope_fwd(*args) == C.DT_ERR_INVALID_ARG and "ctx is NULL" in last_error()
    bad = list(args)
    bad[12] = 96
    assert lib.dt_qk_norm_rope_fwd(*bad) == C.DT_ERR_UNSUPPORTED
    bad = list(args)
    bad[13] = 1000
    assert lib.dt_qk_norm_rope_fwd(*bad) == C.DT_ERR_INVALID_ARG and "stride" in last_error()
    bad = list(args)
    bad[10] = 9000
    assert lib.dt_qk_norm_rope_fwd(*bad) == C.DT_ERR_INVALID_ARG
    assert lib.dt_attn_layer_fwd(None, FAKE, FAKE, 1, 16, None, 0, 0, 0, None) == C.DT_ERR_INVALID_ARG
    assert "layer is NULL" in last_error()
    assert lib.dt_attn_layer_fwd(None, FAKE, FAKE, 1, 9000, None, 0, 0, 0, None) == C.DT_ERR_INVALID_ARG
    assert lib.dt_attn_layer_fwd(None, FAKE, FAKE, 1, 16, None, 3, 0, 0, None) == C.DT_ERR_INVALID_ARG
    assert lib.dt_attn_layer_fwd(None, FAKE, FAKE, 1, 16, None, 0, 0, 2, None) == C.DT_ERR_INVALID_ARG
    lens = (ctypes.c_int32 * 1)(16)
    assert lib.dt_attn_layer_fwd(None, FAKE, FAKE, 1, 16, ctypes.cast(lens, ctypes.c_void_p), 0, 0, 1,
                                 None) == C.DT_ERR_UNSUPPORTED and "seq_lens" in last_error()
    # training entry points: argument checks before any device work
    assert lib.dt_attn_layer_bwd(None, FAKE, FAKE, 1, 16, 0, None) == C.DT_ERR_INVALID_ARG
    assert "layer is NULL" in last_error()
    assert lib.dt_attn_layer_bwd(None, None, FAKE, 1, 16, 0, None) == C.DT_ERR_INVALID_ARG
    assert lib.dt_attn_layer_bwd(None, FAKE, FAKE, 1, 16, 9, None) == C.DT_ERR_INVALID_ARG
    assert lib.dt_attn_layer_step(None, 0.1, None) == C.DT_ERR_INVALID_ARG
    assert lib.dt_attn_layer_zero_grad(None, None) == C.DT_ERR_INVALID_ARG
    assert lib.dt_attn_layer_get_grads(None, None, None, None, None, None, None, 1, None) == C.DT_ERR_INVALID_ARG
    assert lib.dt_attn_layer_get_weights(None, None, None, None, None, None, None, 1, None) == C.DT_ERR_INVALID_ARG
    h = ctypes.c_void_p()
    assert lib.dt_attn_layer_create(None, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 2000, 16, 0,
                                    ctypes.byref(h)) == C.DT_ERR_UNSUPPORTED
    assert lib.dt_ctx_create(-1, ctypes.byref(h)) == C.DT_ERR_INVALID_ARG


def _save_layer(folder, idx, d=256, dtype=np.float32):
    rng = np.random.default_rng(0)
    for n in ("q_proj", "k_proj", "v_proj", "o_proj"):
        np.save(os.path.join(folder, f"model.layers.{idx}.self_attn.{n}.weight.npy"),
                rng.standard_normal((d, d)).astype(dtype))
    for n in ("q_norm", "k_norm"):
        np.save(os.path.join(folder, f"model.layers.{idx}.self_attn.{n}.weight.npy"),
                rng.standard_normal(d).astype(dtype))


def test_npy_loader(tmp_path):
    """dt_attn_layer_load parses the reference's per-layer .npy files before it needs a device."""
    lib = C.lib()
    h = ctypes.c_void_p()
    _save_layer(str(tmp_path), 2)
    # a well-formed folder parses completely; only the missing context stops it
    assert lib.dt_attn_layer_load(None, str(tmp_path).encode(), 2, ctypes.byref(h)) == C.DT_ERR_INVALID_ARG
    assert "ctx is NULL" in last_error()
    assert lib.dt_attn_layer_load(None, str(tmp_path).encode(), 5, ctypes.byref(h)) == C.DT_ERR_IO
    assert "cannot open" in last_error()
    # a Git-LFS pointer in place of the array (what the reference checkout holds)
    p = tmp_path / "model.layers.2.self_attn.q_proj.weight.npy"
    p.write_text("version https://git-lfs.github.com/spec/v1\noid sha256:0\nsize 16777344\n")
    assert lib.dt_attn_layer_load(None, str(tmp_path).encode(), 2, ctypes.byref(h)) == C.DT_ERR_IO
    assert "not a .npy" in last_error()
    f64 = tmp_path / "f64"
    f64.mkdir()
    _save_layer(str(f64), 0, dtype=np.float64)
    assert lib.dt_attn_layer_load(None, str(f64).encode(), 0, ctypes.byref(h)) == C.DT_ERR_IO
    assert "float32" in last_error()
    odd = tmp_path / "odd"
    odd.mkdir()
    _save_layer(str(odd), 0, d=200)
    assert lib.dt_attn_layer_load(None, str(odd).encode(), 0, ctypes.byref(h)) == C.DT_ERR_UNSUPPORTED


def test_cpp_dropin_headers_compile_and_throw():
    sys.path.insert(0, os.path.join(ROOT, "tests", "cpp"))
    import build_dropin as cpp_build

    exe = cpp_build.build()
    r = subprocess.run([str(exe), "cpu"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("OK")
    assert "head_dim 64 != 128" in r.stdout


def test_bench_refuses_multi_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_ctx_option_validation():
    """dt_ctx_set_option rejects a NULL context before touching it (no GPU needed)."""
    lib = C.lib()
    assert lib.dt_ctx_set_option(None, C.DT_OPT_QKV_FUSED, C.DT_QKV_AUTO) == C.DT_ERR_INVALID_ARG
    assert "ctx is NULL" in last_error()


def test_gemm_tune_option_validation():
    lib = C.lib()
    assert lib.dt_ctx_set_option(None, C.DT_OPT_GEMM_TUNE, 1) == C.DT_ERR_INVALID_ARG


def test_bwd_dq_option_validation():
    lib = C.lib()
    assert lib.dt_ctx_set_option(None, C.DT_OPT_BWD_DQ, C.DT_BWD_DQ_FROM_DS) == C.DT_ERR_INVALID_ARG
    assert "ctx is NULL" in last_error()


def _save_model(folder, n_layers=2, vocab=300, hidden=256, d_model=256):
    from dirktensor_amd import synth

    params = synth.model_params(n_layers, vocab, hidden, d_model, seed_base=7700)
    for name, arr in params.items():
        np.save(os.path.join(folder, name + ".npy"), arr.astype(np.float32))
    return params


def test_model_loader_validates_every_file(tmp_path):
    """dt_model_load (the OlmoModel(folder) constructor, OlmoModel.cpp:12-23) checks every file's header and shape
    before it needs a device: a complete folder stops only at the missing context; a Git-LFS pointer, a float64
    file, a wrong shape, a truncated file or a missing block are each reported as DT_ERR_IO."""
    lib = C.lib()
    h = ctypes.c_void_p()
    d = str(tmp_path)
    _save_model(d)
    assert lib.dt_model_load(None, d.encode(), 2, ctypes.byref(h)) == C.DT_ERR_INVALID_ARG
    assert "ctx is NULL" in last_error()
    assert lib.dt_model_load(None, d.encode(), 3, ctypes.byref(h)) == C.DT_ERR_IO  # no block 2
    assert "model.layers.2." in last_error() and "cannot open" in last_error()
    assert lib.dt_model_load(None, d.encode(), 0, ctypes.byref(h)) == C.DT_ERR_INVALID_ARG

    def broken(name, how):
        sub = tmp_path / f"broken_{how}"
        sub.mkdir()
        _save_model(str(sub))
        p = sub / f"{name}.npy"
        if how == "lfs":
            p.write_text("version https://git-lfs.github.com/spec/v1\noid sha256:0\nsize 16777344\n")
        elif how == "f64":
            np.save(p, np.load(p).astype(np.float64))
        elif how == "shape":
            np.save(p, np.load(p)[:, :-1].copy())
        elif how == "trunc":
            p.write_bytes(p.read_bytes()[:-4])
        return str(sub).encode()

    cases = [("model.layers.1.mlp.down_proj.weight", "lfs", "not a .npy"),
             ("model.layers.0.self_attn.q_proj.weight", "f64", "float32"),
             ("model.layers.1.self_attn.o_proj.weight", "shape", "where (256,256,) was expected"),
             ("lm_head.weight", "trunc", "truncated data")]
    for name, how, msg in cases:
        assert lib.dt_model_load(None, broken(name, how), 2, ctypes.byref(h)) == C.DT_ERR_IO, (name, how)
        assert msg in last_error() and name in last_error(), last_error()
