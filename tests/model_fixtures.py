"""Shared model fixtures for oracle and GPU tests.

* ``tiny_*``: the reference's deterministic fixture model
  (crates/orion-models/src/transformer.rs:459-523): weight_matrix(rows, cols,
  seed)[i] = sin(i * 0.37 + seed) * 0.5, hidden 4, 2 q heads / 1 kv head,
  head_dim 2, vocab 8, ffn 8, 16 blocks of 4, norms = 1, tied LM head.
* ``dense_forward_f64``: an independent float64 restatement of the decoder
  forward with *dense* (de-paged) causal attention, used to pin the oracle.
"""
import numpy as np

import oracle as orc


def weight_matrix(rows, cols, seed):
    i = np.arange(rows * cols, dtype=np.float32)
    # Rust: ((i as f32 * 0.37 + seed).sin()) * 0.5, all in f32
    return (np.sin(i * np.float32(0.37) + np.float32(seed)).astype(np.float32)
            * np.float32(0.5)).reshape(rows, cols)


class Spec:
    def __init__(self, L, H, hq, hkv, d, F, V, max_pos=2048, eps=1e-5, theta=10000.0,
                 bias=False, tied=False, num_blocks=16, block_size=4):
        self.L, self.H, self.hq, self.hkv, self.d, self.F, self.V = L, H, hq, hkv, d, F, V
        self.max_pos, self.eps, self.theta = max_pos, eps, theta
        self.bias, self.tied, self.num_blocks, self.block_size = bias, tied, num_blocks, block_size


def tiny_spec(num_layers):
    return Spec(num_layers, 4, 2, 1, 2, 8, 8, max_pos=32, tied=True, num_blocks=16, block_size=4)


def tiny_weights(spec):
    """transformer.rs:486-523."""
    W = {"embed": weight_matrix(spec.V, spec.H, 0.5), "final_norm": np.ones(spec.H, np.float32),
         "lm_head": None, "layers": []}
    qd, kvd = spec.hq * spec.d, spec.hkv * spec.d
    for i in range(spec.L):
        s = float(i)
        W["layers"].append(dict(
            input_norm=np.ones(spec.H, np.float32), q=weight_matrix(qd, spec.H, s + 1.0),
            k=weight_matrix(kvd, spec.H, s + 2.0), v=weight_matrix(kvd, spec.H, s + 3.0),
            o=weight_matrix(spec.H, qd, s + 4.0), post_norm=np.ones(spec.H, np.float32),
            gate=weight_matrix(spec.F, spec.H, s + 5.0), up=weight_matrix(spec.F, spec.H, s + 6.0),
            down=weight_matrix(spec.H, spec.F, s + 7.0), q_bias=None, k_bias=None, v_bias=None))
    return W


def random_weights(spec, rng, std=0.02, bf16=True):
    """N(0, std) weights (optionally rounded to bf16), norms around 1."""
    def mat(r, c):
        w = (rng.standard_normal((r, c)) * std).astype(np.float32)
        return bf16_round(w) if bf16 else w

    def vec(n, base=0.0, scale=std):
        v = (base + rng.standard_normal(n) * scale).astype(np.float32)
        return bf16_round(v) if bf16 else v

    qd, kvd = spec.hq * spec.d, spec.hkv * spec.d
    W = {"embed": mat(spec.V, spec.H), "final_norm": vec(spec.H, 1.0, 0.1),
         "lm_head": None if spec.tied else mat(spec.V, spec.H), "layers": []}
    for _ in range(spec.L):
        W["layers"].append(dict(
            input_norm=vec(spec.H, 1.0, 0.1), q=mat(qd, spec.H), k=mat(kvd, spec.H),
            v=mat(kvd, spec.H), o=mat(spec.H, qd), post_norm=vec(spec.H, 1.0, 0.1),
            gate=mat(spec.F, spec.H), up=mat(spec.F, spec.H), down=mat(spec.H, spec.F),
            q_bias=vec(qd) if spec.bias else None, k_bias=vec(kvd) if spec.bias else None,
            v_bias=vec(kvd) if spec.bias else None))
    return W


def bf16_round(x):
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32) << 16
    return r.view(np.float32)


def oracle_model(spec, W, kv_bf16=False):
    m = orc.OracleTransformer(spec.L, spec.H, spec.hq, spec.hkv, spec.d, spec.F, spec.V,
                              spec.max_pos, spec.eps, spec.theta, spec.bias, spec.tied,
                              spec.num_blocks, spec.block_size, kv_bf16=kv_bf16)
    m.set_weight(orc.W_EMBED, -1, W["embed"])
    m.set_weight(orc.W_FINAL_NORM, -1, W["final_norm"])
    if W["lm_head"] is not None:
        m.set_weight(orc.W_LM_HEAD, -1, W["lm_head"])
    for l, w in enumerate(W["layers"]):
        for key, wid in [("input_norm", orc.W_INPUT_NORM), ("q", orc.W_Q), ("k", orc.W_K),
                         ("v", orc.W_V), ("o", orc.W_O), ("post_norm", orc.W_POST_NORM),
                         ("gate", orc.W_GATE), ("up", orc.W_UP), ("down", orc.W_DOWN),
                         ("q_bias", orc.W_Q_BIAS), ("k_bias", orc.W_K_BIAS),
                         ("v_bias", orc.W_V_BIAS)]:
            if w[key] is not None:
                m.set_weight(wid, l, w[key])
    return m


def dense_forward_f64(spec, W, tokens):
    """Float64 forward of ONE sequence processed from position 0, with dense
    causal attention (no paging, no KV cache).  Returns the last row's logits."""
    n = len(tokens)
    h = W["embed"].astype(np.float64)[np.asarray(tokens)]
    half = spec.d // 2
    i = np.arange(half)
    inv = 1.0 / np.power(float(spec.theta), 2.0 * i / spec.d)
    ang = np.arange(n)[:, None] * inv[None, :]
    cos, sin = np.cos(ang), np.sin(ang)

    def rms(x, w):
        return x / np.sqrt((x ** 2).mean(axis=-1, keepdims=True) + spec.eps) * w

    def rope(x):  # x [n, heads, d]
        x0, x1 = x[..., :half], x[..., half:]
        c, s = cos[:, None, :], sin[:, None, :]
        return np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], axis=-1)

    g = spec.hq // spec.hkv
    mask = np.tril(np.ones((n, n), bool))
    for w in W["layers"]:
        x = rms(h, w["input_norm"])
        q = x @ w["q"].T.astype(np.float64) + (0 if w["q_bias"] is None else w["q_bias"])
        k = x @ w["k"].T.astype(np.float64) + (0 if w["k_bias"] is None else w["k_bias"])
        v = x @ w["v"].T.astype(np.float64) + (0 if w["v_bias"] is None else w["v_bias"])
        q = rope(q.reshape(n, spec.hq, spec.d))
        k = rope(k.reshape(n, spec.hkv, spec.d))
        v = v.reshape(n, spec.hkv, spec.d)
        out = np.empty((n, spec.hq, spec.d))
        for hh in range(spec.hq):
            kh = hh // g
            sc = q[:, hh, :] @ k[:, kh, :].T / np.sqrt(spec.d)
            sc = np.where(mask, sc, -np.inf)
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            p /= p.sum(axis=1, keepdims=True)
            out[:, hh, :] = p @ v[:, kh, :]
        h = h + out.reshape(n, -1) @ w["o"].T.astype(np.float64)
        x = rms(h, w["post_norm"])
        gt = x @ w["gate"].T.astype(np.float64)
        up = x @ w["up"].T.astype(np.float64)
        h = h + (gt / (1 + np.exp(-gt)) * up) @ w["down"].T.astype(np.float64)
    h = rms(h, W["final_norm"])
    head = W["embed"] if W["lm_head"] is None else W["lm_head"]
    return h[-1] @ head.T.astype(np.float64)
