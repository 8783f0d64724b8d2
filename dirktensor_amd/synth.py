"""Seeded synthetic workloads for the attention path.

Every tensor is drawn from its own seed with a counter-based splitmix64 stream,
turned into standard normals by fp64 Box-Muller and cast to fp32, in row-major
linear order.  bf16 inputs are the round-to-nearest-even bf16 of the same fp32
draws, so the bf16 and fp32 modes see the same underlying values.

The reference loads trained OLMo-2 weights from .npy files
(OlmoAttention.cpp:39-53); those files are Git-LFS pointers in the reference
checkout, so every workload here uses seeded random weights instead:
projection weights ~ N(0, 0.02), norm weights ~ 1 + N(0, 0.01).
"""

from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int) -> np.ndarray:
    """The first ``n`` outputs of splitmix64 seeded with ``seed`` (uint64 array)."""
    with np.errstate(over="ignore"):
        ctr = np.arange(1, n + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + ctr * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        z = z ^ (z >> np.uint64(31))
    return z


def uniform01(seed: int, n: int) -> np.ndarray:
    """``n`` fp64 uniforms in [0, 1) (top 53 bits of splitmix64)."""
    return (splitmix64(seed, n) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def normal(seed: int, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """fp32 array of the given shape ~ N(mean, std^2) from ``seed`` (Box-Muller in fp64)."""
    n = int(np.prod(shape)) if len(shape) else 1
    pairs = (n + 1) // 2
    u = uniform01(seed, 2 * pairs)
    u1 = 1.0 - u[0::2]  # (0, 1]
    u2 = u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * pairs, dtype=np.float64)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    return (mean + std * z[:n]).astype(np.float32).reshape(shape)


def uniform_int(seed: int, n: int, lo: int, hi: int) -> np.ndarray:
    """``n`` int64 values uniform in [lo, hi] (inclusive)."""
    u = uniform01(seed, n)
    return (lo + np.floor(u * (hi - lo + 1))).astype(np.int64)


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16, returned as uint16 bit patterns."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    rounded[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return rounded


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """fp32 values rounded to the nearest bf16 (returned as fp32)."""
    return bf16_bits_to_f32(to_bf16_bits(x)).reshape(np.shape(x))


# ---------------------------------------------------------------------------
# Named workloads (seeds are part of the workload definition)

QKV_SEEDS = (1001, 1002, 1003)


def qkv(B: int, T: int, H: int = 16, D: int = 128, seeds=QKV_SEEDS):
    """Q, K, V [B, T, H, D] fp32 ~ N(0, 1) (attention-core workloads)."""
    return tuple(normal(s, (B, T, H, D)) for s in seeds)


def ragged_lengths(B: int = 8, lo: int = 64, hi: int = 2048, seed: int = 4001) -> np.ndarray:
    """Per-sequence lengths uniform in [lo, hi] for the batched ragged prefill workload."""
    return uniform_int(seed, B, lo, hi).astype(np.int32)


def attention_layer_weights(d_model: int = 2048, seed_base: int = 2011, norm_seeds=(2021, 2022)):
    """Wq, Wk, Wv, Wo [d, d] ~ N(0, 0.02) ([out, in] like torch Linear); q/k norm ~ 1 + N(0, 0.01)."""
    ws = [normal(seed_base + i, (d_model, d_model), 0.0, 0.02) for i in range(4)]
    qn = normal(norm_seeds[0], (d_model,), 1.0, 0.01)
    kn = normal(norm_seeds[1], (d_model,), 1.0, 0.01)
    return dict(wq=ws[0], wk=ws[1], wv=ws[2], wo=ws[3], q_norm=qn, k_norm=kn)


def layer_input(B: int = 1, T: int = 512, d_model: int = 2048, seed: int = 2001) -> np.ndarray:
    return normal(seed, (B, T, d_model))


MODEL_LAYER_PARAMS = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                      "self_attn.q_norm", "self_attn.k_norm", "post_attention_layernorm", "mlp.gate_proj",
                      "mlp.up_proj", "mlp.down_proj", "post_feedforward_layernorm")


def model_params(n_layers: int = 16, vocab: int = 100352, hidden: int = 8192, d_model: int = 2048,
                 seed_base: int = 5100) -> dict:
    """Seeded OLMo-2 weights keyed by the reference's .npy file stems (OlmoModel.cpp:12-22,
    OlmoBlock.cpp:5-11, OlmoMlp.cpp:9-24, OlmoAttention.cpp:39-53). Matrices ~ N(0, 0.02) rounded to
    bf16-representable fp32 (so both modes see the same weights), norm weights ~ 1 + N(0, 0.01); the
    k-th array in creation order uses seed seed_base + k."""
    shapes = {"self_attn.q_proj": (d_model, d_model), "self_attn.k_proj": (d_model, d_model),
              "self_attn.v_proj": (d_model, d_model), "self_attn.o_proj": (d_model, d_model),
              "self_attn.q_norm": (d_model,), "self_attn.k_norm": (d_model,), "post_attention_layernorm": (d_model,),
              "mlp.gate_proj": (hidden, d_model), "mlp.up_proj": (hidden, d_model), "mlp.down_proj": (d_model, hidden),
              "post_feedforward_layernorm": (d_model,)}
    out = {}
    k = 0

    def draw(shape):
        nonlocal k
        seed = seed_base + k
        k += 1
        if len(shape) == 1:
            return normal(seed, shape, 1.0, 0.01)
        return round_bf16(normal(seed, shape, 0.0, 0.02))

    out["model.embed_tokens.weight"] = draw((vocab, d_model))
    for i in range(n_layers):
        for name in MODEL_LAYER_PARAMS:
            out[f"model.layers.{i}.{name}.weight"] = draw(shapes[name])
    out["model.norm.weight"] = draw((d_model,))
    out["lm_head.weight"] = draw((vocab, d_model))
    return out


def model_param_shapes(n_layers: int = 16, vocab: int = 100352, hidden: int = 8192, d_model: int = 2048) -> list:
    """(name, shape) of every OLMo-2 parameter in creation order (the order model_params draws them in)."""
    d = d_model
    shapes = {"self_attn.q_proj": (d, d), "self_attn.k_proj": (d, d), "self_attn.v_proj": (d, d),
              "self_attn.o_proj": (d, d), "self_attn.q_norm": (d,), "self_attn.k_norm": (d,),
              "post_attention_layernorm": (d,), "mlp.gate_proj": (hidden, d), "mlp.up_proj": (hidden, d),
              "mlp.down_proj": (d, hidden), "post_feedforward_layernorm": (d,)}
    names = [("model.embed_tokens.weight", (vocab, d))]
    for i in range(n_layers):
        names += [(f"model.layers.{i}.{n}.weight", shapes[n]) for n in MODEL_LAYER_PARAMS]
    names += [("model.norm.weight", (d,)), ("lm_head.weight", (vocab, d))]
    return names


def device_model_params(device, n_layers: int = 16, vocab: int = 100352, hidden: int = 8192, d_model: int = 2048,
                        seed: int = 5100):
    """The OLMo-2-1B-sized weights drawn on the GPU (numpy's seeded draw of 1.48 B values takes minutes):
    yields (name, fp32 device tensor) in creation order from one seeded torch.Generator on ``device``;
    matrices ~ N(0, 0.02) rounded to bf16-representable fp32, norm weights ~ 1 + N(0, 0.01). The same seed
    gives the same weights on the same torch build."""
    import torch

    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    for name, shape in model_param_shapes(n_layers, vocab, hidden, d_model):
        if len(shape) == 1:
            w = 1.0 + 0.01 * torch.randn(shape, generator=gen, device=device)
        else:
            w = (0.02 * torch.randn(shape, generator=gen, device=device)).bfloat16().float()
        yield name, w


def model_tokens(B: int = 1, T: int = 2048, vocab: int = 100352, seed: int = 5001) -> np.ndarray:
    """Token ids ~ U[0, vocab) for the end-to-end workloads, int32 [B, T]."""
    return uniform_int(seed, B * T, 0, vocab - 1).astype(np.int32).reshape(B, T)
