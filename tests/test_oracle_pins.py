"""Pins of the CPU oracle (CPU only).

The reference's own checks of this path cannot run anywhere in this pipeline
(test_olmo_model.cpp:48-70 and tests/test_backward.py:56-86 need trained
weights that are Git-LFS pointers, plus network access), so the oracle is
pinned against things that fix the answer independently of its code:

* an fp64 full-softmax attention written here in numpy (not tiled, no online
  rescale) and torch's scaled_dot_product_attention in fp64;
* brute force over every (query, key) pair at T <= 8;
* closed forms: row 0 returns V[0] with l = 1 and m = scale * q0.k0; Q = 0
  gives the running mean of V with m = 0 and l = t + 1; causality;
* HF transformers' OLMo-2 building blocks (a separate implementation of the
  same model): rotate_half / apply_rotary_pos_emb, Olmo2RotaryEmbedding,
  Olmo2RMSNorm and the whole Olmo2Attention layer, run in fp64 with the
  oracle's fp64-derived RoPE tables;
* torch.nn.functional.rms_norm in fp64, and RoPE invariants (identity at
  t = 0, pair norms preserved, scores depend only on t1 - t2).

* model: HF's Olmo2ForCausalLM (2 layers) in fp64 for the whole forward,
  torch's F.silu MLP, and F.cross_entropy(ignore_index) with its autograd
  gradient for ce_loss and main.cpp's loss gradient;
* backward: torch autograd in fp64 through scaled_dot_product_attention,
  F.rms_norm, HF's apply_rotary_pos_emb and the whole Olmo2Attention layer
  (d_x and all six weight gradients); central finite differences of a numpy
  fp64 attention; the adjoint identity <rope(x), g> = <x, rope_bwd(g)>; and
  the row-stochastic invariants sum_k dK = 0, sum_k dV = sum_q dO.

test_planted_mistakes_are_caught then plants each of the oracle's known
mistakes (oracle_set_mutation) and checks that at least one pin fails.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from dirktensor_amd import synth

SCALE = float(np.float32(1.0) / np.sqrt(np.float32(128.0)))


# ----------------------------------------------------------------- independent formulations
def textbook_attention_f64(Q, K, V, scale, causal=True):
    q, k, v = (np.asarray(x, np.float64).transpose(0, 2, 1, 3) for x in (Q, K, V))  # B,H,T,D
    s = scale * (q @ k.transpose(0, 1, 3, 2))
    T = s.shape[-1]
    if causal:
        s = np.where(np.triu(np.ones((T, T), bool), 1), -np.inf, s)
    m = s.max(-1)
    p = np.exp(s - m[..., None])
    l = p.sum(-1)
    o = (p @ v) / l[..., None]
    return o.transpose(0, 2, 1, 3), m.transpose(0, 2, 1), l.transpose(0, 2, 1)


def brute_force_attention(Q, K, V, scale):
    B, T, H, D = Q.shape
    O = np.zeros((B, T, H, D))
    m = np.zeros((B, T, H))
    l = np.zeros((B, T, H))
    for b in range(B):
        for h in range(H):
            for t in range(T):
                scores = [scale * sum(float(Q[b, t, h, d]) * float(K[b, j, h, d]) for d in range(D))
                          for j in range(t + 1)]
                mx = max(scores)
                w = [np.exp(x - mx) for x in scores]
                m[b, t, h], l[b, t, h] = mx, sum(w)
                for j in range(t + 1):
                    O[b, t, h] += w[j] * V[b, j, h].astype(np.float64)
                O[b, t, h] /= l[b, t, h]
    return O, m, l


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def hf_config():
    from transformers import Olmo2Config

    return Olmo2Config(hidden_size=2048, intermediate_size=8192, num_attention_heads=16, num_key_value_heads=16,
                       max_position_embeddings=8192, rms_norm_eps=1e-6, attention_bias=False,
                       rope_parameters={"rope_type": "default", "rope_theta": 500000.0})


# ----------------------------------------------------------------- pins (return True when they hold)
def pin_flash_textbook(causal=True):
    Q, K, V = synth.qkv(1, 300, 2, seeds=(41, 42, 43))  # 300 > 256 exercises the tile-to-tile rescale
    O, m, l = oracle.flash_attention_forward(Q, K, V, SCALE, causal)
    Ot, mt, lt = textbook_attention_f64(Q, K, V, SCALE, causal)
    return rel(O, Ot) <= 1e-5 and np.max(np.abs(m - mt)) <= 1e-5 * np.max(np.abs(mt)) and rel(l, lt) <= 1e-5


def pin_flash_sdpa():
    Q, K, V = synth.qkv(2, 280, 3, seeds=(51, 52, 53))
    O, _, _ = oracle.flash_attention_forward(Q, K, V, SCALE)
    q, k, v = (torch.from_numpy(x).double().transpose(1, 2) for x in (Q, K, V))
    ref = F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=SCALE).transpose(1, 2).numpy()
    return rel(O, ref) <= 1e-5


def pin_flash_bruteforce():
    Q, K, V = synth.qkv(1, 8, 2, seeds=(61, 62, 63))
    O, m, l = oracle.flash_attention_forward(Q, K, V, SCALE)
    Ob, mb, lb = brute_force_attention(Q, K, V, SCALE)
    return rel(O, Ob) <= 1e-5 and np.max(np.abs(m - mb)) <= 1e-5 and rel(l, lb) <= 1e-5


def pin_flash_closed_forms():
    Q, K, V = synth.qkv(1, 260, 2, seeds=(71, 72, 73))
    O, m, l = oracle.flash_attention_forward(Q, K, V, SCALE)
    ok = np.array_equal(O[0, 0], V[0, 0]) and np.all(l[0, 0] == 1.0)
    s00 = SCALE * np.sum(Q[0, 0].astype(np.float64) * K[0, 0], axis=-1)
    ok &= np.max(np.abs(m[0, 0] - s00)) <= 1e-5 * max(1.0, np.max(np.abs(s00)))
    Z = np.zeros_like(Q)
    Oz, mz, lz = oracle.flash_attention_forward(Z, K, V, SCALE)
    mean = np.cumsum(V.astype(np.float64), axis=1) / np.arange(1, 261)[None, :, None, None]
    ok &= rel(Oz, mean) <= 1e-5 and np.all(mz == 0.0)
    ok &= np.max(np.abs(lz[0, :, 0] - np.arange(1, 261))) <= 1e-3
    return bool(ok)


def pin_flash_causality():
    Q, K, V = synth.qkv(1, 300, 2, seeds=(81, 82, 83))
    O, _, _ = oracle.flash_attention_forward(Q, K, V, SCALE)
    K2, V2 = K.copy(), V.copy()
    K2[:, 151:] += 1.0
    V2[:, 151:] -= 2.0
    O2, _, _ = oracle.flash_attention_forward(Q, K2, V2, SCALE)
    return bool(np.array_equal(O[:, :151], O2[:, :151]) and not np.array_equal(O[:, 151:], O2[:, 151:]))


def pin_rope_hf():
    from transformers.models.olmo2.modeling_olmo2 import apply_rotary_pos_emb

    s, c = oracle.rope_tables(64)
    x = synth.normal(91, (2, 64, 3, 128))
    y = synth.normal(92, (2, 64, 3, 128))
    ox, oy = oracle.apply_rope(x, s, c), oracle.apply_rope(y, s, c)
    cos = torch.from_numpy(c).double()[None]  # [1, T, D]
    sin = torch.from_numpy(s).double()[None]
    hx, hy = apply_rotary_pos_emb(torch.from_numpy(x).double(), torch.from_numpy(y).double(), cos, sin,
                                  unsqueeze_dim=2)
    return rel(ox, hx.numpy()) <= 1e-6 and rel(oy, hy.numpy()) <= 1e-6


def pin_rope_tables():
    from transformers.models.olmo2.modeling_olmo2 import Olmo2RotaryEmbedding

    s, c = oracle.rope_tables(8192)
    cos, sin = Olmo2RotaryEmbedding(hf_config())(torch.zeros(1), torch.arange(8192)[None])
    # HF evaluates the angles in fp32 (a ~1e-4 difference at t ~ 8k); the reference, and the oracle, in fp64.
    ok = np.max(np.abs(c - cos[0].numpy())) <= 2e-3 and np.max(np.abs(s - sin[0].numpy())) <= 2e-3
    t = np.arange(8192, dtype=np.float64)
    ok &= np.array_equal(s[:, 0], np.sin(t).astype(np.float32)) and np.array_equal(c[:, 64], np.cos(t).astype(np.float32))
    ok &= np.array_equal(s[:, :64], s[:, 64:]) and np.array_equal(c[:, :64], c[:, 64:])
    inv_last = 1.0 / 500000.0 ** (126.0 / 128.0)
    ok &= np.array_equal(s[:, 63], np.sin(t * inv_last).astype(np.float32))
    return bool(ok)


def pin_rope_invariants():
    s, c = oracle.rope_tables(512)
    x = synth.normal(93, (1, 512, 1, 128))
    r = oracle.apply_rope(x, s, c)
    ok = np.array_equal(r[0, 0], x[0, 0])  # t = 0: cos = 1, sin = 0
    n0 = x[..., :64] ** 2 + x[..., 64:] ** 2
    n1 = r[..., :64].astype(np.float64) ** 2 + r[..., 64:].astype(np.float64) ** 2
    ok &= np.max(np.abs(n1 - n0) / np.maximum(n0, 1e-3)) <= 1e-5
    q = np.broadcast_to(synth.normal(94, (1, 1, 1, 128)), (1, 512, 1, 128)).copy()
    k = np.broadcast_to(synth.normal(95, (1, 1, 1, 128)), (1, 512, 1, 128)).copy()
    rq, rk = oracle.apply_rope(q, s, c).astype(np.float64), oracle.apply_rope(k, s, c).astype(np.float64)
    d1 = np.sum(rq[0, 300, 0] * rk[0, 290, 0])
    d2 = np.sum(rq[0, 110, 0] * rk[0, 100, 0])
    ok &= abs(d1 - d2) <= 1e-4 * max(1.0, abs(d1))
    return bool(ok)


def pin_rmsnorm_torch():
    w = synth.normal(96, (2048,), 1.0, 0.01)
    ok = True
    for std in (1.0, 1e-3):  # at std 1e-3 the mean square is ~1e-6, comparable to eps
        x = synth.normal(97, (5, 2048), 0.0, std)
        y, rms = oracle.rmsnorm_forward(x, w)
        ref = F.rms_norm(torch.from_numpy(x).double(), (2048,), torch.from_numpy(w).double(), eps=1e-6).numpy()
        ok &= rel(y, ref) <= 1e-6
        ok &= rel(rms, np.sqrt(np.mean(x.astype(np.float64) ** 2, axis=-1) + 1e-6)) <= 1e-6
    return bool(ok)


def pin_rmsnorm_hf():
    from transformers.models.olmo2.modeling_olmo2 import Olmo2RMSNorm

    w = synth.normal(98, (2048,), 1.0, 0.01)
    x = synth.normal(99, (3, 7, 2048), 0.0, 2.0)
    n = Olmo2RMSNorm(2048, 1e-6)
    with torch.no_grad():
        n.weight.copy_(torch.from_numpy(w))
        ref = n(torch.from_numpy(x)).numpy()
    y, _ = oracle.rmsnorm_forward(x, w)
    big, _ = oracle.rmsnorm_forward(1000.0 * x, w)  # scale invariance (eps negligible)
    return rel(y, ref) <= 2e-6 and rel(big, y) <= 2e-6


def pin_layer_hf(T=48):
    from transformers.models.olmo2.modeling_olmo2 import Olmo2Attention

    w = synth.attention_layer_weights()
    x = synth.normal(2301, (1, T, 2048))
    out = oracle.attention_layer_forward(x, w["wq"], w["wk"], w["wv"], w["wo"], w["q_norm"], w["k_norm"])
    cfg = hf_config()
    cfg._attn_implementation = "eager"
    attn = Olmo2Attention(cfg, 0).double()
    with torch.no_grad():
        attn.q_proj.weight.copy_(torch.from_numpy(w["wq"]))
        attn.k_proj.weight.copy_(torch.from_numpy(w["wk"]))
        attn.v_proj.weight.copy_(torch.from_numpy(w["wv"]))
        attn.o_proj.weight.copy_(torch.from_numpy(w["wo"]))
        attn.q_norm.weight.copy_(torch.from_numpy(w["q_norm"]))
        attn.k_norm.weight.copy_(torch.from_numpy(w["k_norm"]))
        s, c = oracle.rope_tables(T)
        pe = (torch.from_numpy(c).double()[None], torch.from_numpy(s).double()[None])
        mask = torch.triu(torch.full((T, T), float("-inf"), dtype=torch.float64), 1)[None, None]
        ref, _ = attn(torch.from_numpy(x).double(), pe, mask)
    return rel(out, ref.numpy()) <= 1e-4


# ----------------------------------------------------------------- backward pins
def _fwd_bwd(Q, K, V, G, causal=True):
    O, m, l = oracle.flash_attention_forward(Q, K, V, SCALE, causal)
    return O, oracle.flash_attention_backward(G, O, m, l, Q, K, V, SCALE, causal)


def _autograd_attention(Q, K, V, G, causal=True):
    q, k, v = (torch.from_numpy(np.asarray(x, np.float64)).transpose(1, 2).requires_grad_() for x in (Q, K, V))
    o = F.scaled_dot_product_attention(q, k, v, is_causal=causal, scale=SCALE).transpose(1, 2)
    (o * torch.from_numpy(np.asarray(G, np.float64))).sum().backward()
    return [t.grad.transpose(1, 2).numpy() for t in (q, k, v)]


def pin_flash_bwd_autograd(causal=True):
    Q, K, V = synth.qkv(1, 300, 2, seeds=(141, 142, 143))  # 300 > 256: crosses the reference's block edge
    G = synth.normal(144, Q.shape)
    _, grads = _fwd_bwd(Q, K, V, G, causal)
    ref = _autograd_attention(Q, K, V, G, causal)
    return all(rel(a, b) <= 1e-4 for a, b in zip(grads, ref))


def pin_flash_bwd_finite_difference():
    """Central differences of L = sum(O * G) in fp64 (numpy textbook attention), no autograd."""
    Q, K, V = synth.qkv(1, 6, 1, seeds=(151, 152, 153))
    G = synth.normal(154, Q.shape)
    _, (dQ, dK, dV) = _fwd_bwd(Q, K, V, G)
    X = [np.asarray(a, np.float64) for a in (Q, K, V)]

    def loss(xs):
        o, _, _ = textbook_attention_f64(*xs, SCALE)
        return float(np.sum(o * G))

    ok = True
    rng = np.random.default_rng(155)
    for which, grad in enumerate((dQ, dK, dV)):
        for _ in range(6):
            idx = (0, int(rng.integers(6)), 0, int(rng.integers(128)))
            h = 1e-5
            xp = [a.copy() for a in X]
            xm = [a.copy() for a in X]
            xp[which][idx] += h
            xm[which][idx] -= h
            fd = (loss(xp) - loss(xm)) / (2 * h)
            ok &= abs(fd - float(grad[idx])) <= 1e-4 * max(1.0, abs(fd))
    return bool(ok)


def pin_flash_bwd_invariants():
    """Rows of P sum to 1, so the keys' dK sum to 0 and the keys' dV sum to the queries' dO sum."""
    Q, K, V = synth.qkv(1, 280, 2, seeds=(161, 162, 163))
    G = synth.normal(164, Q.shape)
    _, (dQ, dK, dV) = _fwd_bwd(Q, K, V, G)
    sk = np.abs(dK.astype(np.float64).sum(axis=1)).max() / np.abs(dK).max()
    sv = rel(dV.astype(np.float64).sum(axis=1), G.astype(np.float64).sum(axis=1))
    return sk <= 1e-4 and sv <= 1e-5


def pin_rope_bwd_adjoint():
    """apply_rope_backward is the transpose of apply_rope: <rope(x), g> = <x, rope_bwd(g)>, per (t, h)."""
    s, c = oracle.rope_tables(300)
    x = synth.normal(171, (2, 300, 3, 128))
    g = synth.normal(172, (2, 300, 3, 128))
    lhs = np.sum(oracle.apply_rope(x, s, c).astype(np.float64) * g, axis=-1)
    rhs = np.sum(x.astype(np.float64) * oracle.apply_rope_backward(g, s, c), axis=-1)
    back = oracle.apply_rope_backward(oracle.apply_rope(x, s, c), s, c)  # a rotation: the inverse too
    return rel(lhs, rhs) <= 1e-5 and rel(back, x) <= 1e-5


def pin_rope_bwd_autograd():
    from transformers.models.olmo2.modeling_olmo2 import apply_rotary_pos_emb

    s, c = oracle.rope_tables(64)
    x = torch.from_numpy(synth.normal(173, (1, 64, 2, 128))).double().requires_grad_()
    g = synth.normal(174, (1, 64, 2, 128))
    y, _ = apply_rotary_pos_emb(x, x.detach(), torch.from_numpy(c).double()[None], torch.from_numpy(s).double()[None],
                                unsqueeze_dim=2)
    (y * torch.from_numpy(g).double()).sum().backward()
    return rel(oracle.apply_rope_backward(g, s, c), x.grad.numpy()) <= 1e-6


def pin_rmsnorm_bwd_autograd():
    w = synth.normal(181, (2048,), 1.0, 0.01)
    ok = True
    for std in (1.0, 1e-3):
        x = synth.normal(182, (5, 2048), 0.0, std)
        g = synth.normal(183, (5, 2048))
        y, rms = oracle.rmsnorm_forward(x, w)
        dx, dw = oracle.rmsnorm_backward(g, y, rms, w)
        xt = torch.from_numpy(x).double().requires_grad_()
        wt = torch.from_numpy(w).double().requires_grad_()
        (F.rms_norm(xt, (2048,), wt, eps=1e-6) * torch.from_numpy(g).double()).sum().backward()
        ok &= rel(dx, xt.grad.numpy()) <= 1e-5 and rel(dw, wt.grad.numpy()) <= 1e-5
    return bool(ok)


def pin_layer_bwd_hf(T=40):
    """d_x and all six weight gradients against torch autograd through HF's Olmo2Attention in fp64."""
    from transformers.models.olmo2.modeling_olmo2 import Olmo2Attention

    w = synth.attention_layer_weights()
    x = synth.normal(2401, (1, T, 2048))
    g = synth.normal(2402, (1, T, 2048))
    d_x, grads = oracle.attention_layer_backward(x, w["wq"], w["wk"], w["wv"], w["wo"], w["q_norm"], w["k_norm"], g)
    cfg = hf_config()
    cfg._attn_implementation = "eager"
    attn = Olmo2Attention(cfg, 0).double()
    names = {"wq": attn.q_proj, "wk": attn.k_proj, "wv": attn.v_proj, "wo": attn.o_proj,
             "q_norm": attn.q_norm, "k_norm": attn.k_norm}
    with torch.no_grad():
        for k, mod in names.items():
            mod.weight.copy_(torch.from_numpy(w[k]))
    s, c = oracle.rope_tables(T)
    pe = (torch.from_numpy(c).double()[None], torch.from_numpy(s).double()[None])
    mask = torch.triu(torch.full((T, T), float("-inf"), dtype=torch.float64), 1)[None, None]
    xt = torch.from_numpy(x).double().requires_grad_()
    out, _ = attn(xt, pe, mask)
    (out * torch.from_numpy(g).double()).sum().backward()
    ok = rel(d_x, xt.grad.numpy()) <= 1e-4
    for k, mod in names.items():
        ok &= rel(grads[k], mod.weight.grad.numpy()) <= 1e-4
    return bool(ok)


# ----------------------------------------------------------------- model pins
def _small_model(n_layers=2, vocab=300, hidden=512):
    return synth.model_params(n_layers=n_layers, vocab=vocab, hidden=hidden, seed_base=5900)


def pin_mlp_torch():
    p = _small_model(1)
    x = synth.normal(3001, (20, 2048))
    wg, wu, wd = (p[f"model.layers.0.mlp.{n}_proj.weight"] for n in ("gate", "up", "down"))
    out = oracle.mlp_forward(x, wg, wu, wd)
    xt, g, u, d = (torch.from_numpy(a).double() for a in (x, wg, wu, wd))
    ref = (F.silu(xt @ g.T) * (xt @ u.T)) @ d.T
    return rel(out, ref.numpy()) <= 1e-5


def _hf_model(p, n_layers, vocab, hidden):
    from transformers import Olmo2ForCausalLM

    cfg = hf_config()
    cfg.num_hidden_layers = n_layers
    cfg.vocab_size = vocab
    cfg.intermediate_size = hidden
    cfg.tie_word_embeddings = False
    cfg._attn_implementation = "eager"
    model = Olmo2ForCausalLM(cfg).double().eval()
    sd = {k: torch.from_numpy(v).double() for k, v in p.items()}
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected and all("rotary" in m for m in missing), (missing, unexpected)
    return model


def pin_model_hf():
    """OlmoModel::forward against HF's Olmo2ForCausalLM (post-norm OLMo-2) in fp64, 2 layers."""
    n_layers, vocab, hidden, T = 2, 300, 512, 24
    p = _small_model(n_layers, vocab, hidden)
    tok = synth.model_tokens(2, T, vocab, seed=5902)
    logits = oracle.model_forward(tok, p)
    with torch.no_grad():
        ref = _hf_model(p, n_layers, vocab, hidden)(torch.from_numpy(tok).long()).logits.numpy()
    return rel(logits, ref) <= 1e-4


def pin_model_bwd_hf():
    """OlmoModel::backward: every parameter gradient against torch autograd through HF's Olmo2ForCausalLM."""
    n_layers, vocab, hidden, T = 2, 300, 512, 16
    p = _small_model(n_layers, vocab, hidden)
    tok = synth.model_tokens(1, T, vocab, seed=5903)
    G = synth.normal(5904, (1, T, vocab))
    grads = oracle.model_backward(tok, p, G)
    model = _hf_model(p, n_layers, vocab, hidden)
    (model(torch.from_numpy(tok).long()).logits * torch.from_numpy(G).double()).sum().backward()
    named = dict(model.named_parameters())
    return all(rel(grads[k], named[k].grad.numpy()) <= 1e-4 for k in p)


def pin_ce_torch():
    """ce_loss and main.cpp's gradient against F.cross_entropy(ignore_index) and its autograd in fp64."""
    B, T, V, pad = 3, 17, 50, 7
    logits = synth.normal(3101, (B, T, V), 0.0, 3.0)
    tok = synth.model_tokens(B, T, V, seed=3102)
    tok[1, 9:] = pad  # a right-padded sequence (main.cpp:46-57)
    tok[2, 4] = pad
    loss, g = oracle.ce_loss(logits, tok, pad, with_grad=True)
    lt = torch.from_numpy(logits).double().requires_grad_()
    ref = F.cross_entropy(lt[:, :-1].reshape(-1, V), torch.from_numpy(tok[:, 1:]).long().reshape(-1), ignore_index=pad)
    ref.backward()
    return abs(loss - ref.item()) <= 1e-5 * abs(ref.item()) and rel(g, lt.grad.numpy()) <= 1e-5


def pin_ce_no_targets():
    """With no target at all (every next token ignored, or T = 1) the reference divides 0 by 0
    (CrossEntropyLoss.cpp:40, main.cpp:88): loss NaN and every gradient element NaN. torch's mean over zero
    terms is NaN as well."""
    B, T, V, pad = 2, 9, 30, 4
    logits = synth.normal(3103, (B, T, V))
    tok = np.full((B, T), pad, np.int32)
    tok[:, 0] = 1  # only position 0 is a real token; it is never a target
    loss, g = oracle.ce_loss(logits, tok, pad, with_grad=True)
    ref = F.cross_entropy(torch.from_numpy(logits[:, :-1]).double().reshape(-1, V),
                          torch.from_numpy(tok[:, 1:]).long().reshape(-1), ignore_index=pad)
    loss1, g1 = oracle.ce_loss(logits[:, :1], tok[:, :1], pad, with_grad=True)  # T = 1: no position has a target
    return (np.isnan(loss) and np.isnan(ref.item()) and bool(np.all(np.isnan(g))) and np.isnan(loss1)
            and bool(np.all(np.isnan(g1))))


PINS = {
    "flash_textbook_causal": lambda: pin_flash_textbook(True),
    "flash_textbook_full": lambda: pin_flash_textbook(False),
    "flash_sdpa": pin_flash_sdpa,
    "flash_bruteforce": pin_flash_bruteforce,
    "flash_closed_forms": pin_flash_closed_forms,
    "flash_causality": pin_flash_causality,
    "rope_hf": pin_rope_hf,
    "rope_tables": pin_rope_tables,
    "rope_invariants": pin_rope_invariants,
    "rmsnorm_torch": pin_rmsnorm_torch,
    "rmsnorm_hf": pin_rmsnorm_hf,
    "layer_hf": pin_layer_hf,
    "flash_bwd_autograd_causal": lambda: pin_flash_bwd_autograd(True),
    "flash_bwd_autograd_full": lambda: pin_flash_bwd_autograd(False),
    "flash_bwd_finite_difference": pin_flash_bwd_finite_difference,
    "ce_no_targets": pin_ce_no_targets,
    "flash_bwd_invariants": pin_flash_bwd_invariants,
    "rope_bwd_adjoint": pin_rope_bwd_adjoint,
    "rope_bwd_autograd": pin_rope_bwd_autograd,
    "rmsnorm_bwd_autograd": pin_rmsnorm_bwd_autograd,
    "layer_bwd_hf": pin_layer_bwd_hf,
    "mlp_torch": pin_mlp_torch,
    "model_hf": pin_model_hf,
    "model_bwd_hf": pin_model_bwd_hf,
    "ce_torch": pin_ce_torch,
}


@pytest.mark.parametrize("name", sorted(PINS))
def test_pin_holds(name):
    assert PINS[name](), f"oracle pin {name} failed"


# mutation -> the pins expected to catch it
MUTATIONS = {
    1: ["flash_textbook_causal", "flash_textbook_full"],  # beta dropped from the online rescale
    2: ["flash_closed_forms", "flash_bruteforce"],        # diagonal masked
    3: ["rope_hf", "layer_hf"],                           # sin sign flipped
    4: ["rope_hf", "rope_invariants"],                    # pairs (d, d+1)
    5: ["rmsnorm_torch", "layer_hf"],                     # per-head norm
    6: ["rmsnorm_torch"],                                 # eps dropped
    7: ["flash_textbook_causal", "flash_sdpa"],           # scale dropped
    8: ["flash_bwd_autograd_causal", "flash_bwd_finite_difference", "flash_bwd_invariants"],  # D dropped
    9: ["rope_bwd_adjoint", "rope_bwd_autograd", "layer_bwd_hf"],                            # forward rotation
    10: ["rmsnorm_bwd_autograd", "layer_bwd_hf"],                                            # c term dropped
    11: ["flash_bwd_autograd_causal", "flash_bwd_finite_difference"],                        # 1 / l dropped
    12: ["mlp_torch", "model_hf", "model_bwd_hf"],                                           # SiLU without sigmoid
    13: ["model_hf"],                                                                         # pre-norm blocks
    14: ["ce_torch"],                                                                         # pad targets counted
}


@pytest.mark.parametrize("mut", sorted(MUTATIONS))
def test_planted_mistakes_are_caught(mut):
    with oracle.mutation(mut):
        failing = [n for n in MUTATIONS[mut] if not PINS[n]()]
    assert failing == MUTATIONS[mut], f"mutation {mut}: only {failing} of {MUTATIONS[mut]} caught it"
    assert oracle.lib().oracle_get_mutation() == 0
