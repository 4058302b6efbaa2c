"""Float64 numpy evaluation of the encoder, written from the architecture's
mathematics (post-LN BERT / Nomic-style blocks) with exact exp / tanh.

Used only to pin the C oracle: the oracle in its exact-math mode must agree
with this to float32 rounding, so a transposed operand, a wrong head slice, a
misplaced residual or a wrong RoPE pairing in the oracle shows up as a gross
mismatch.  Vectorised over heads and sequences, unlike the oracle's loops.
"""
import numpy as np


def layer_norm(x, g, b, eps):
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * g + b


def gelu_tanh(x):
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


def rope_rotate(x, base):
    """x: [L, heads, d]; rotate-half with theta_i = pos * base^(-2i/d)."""
    L, _, d = x.shape
    half = d // 2
    inv = base ** (-2.0 * np.arange(half) / d)
    ang = np.arange(L)[:, None] * inv[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c], axis=-1)


def encode_sequence(cfg, W, ids):
    """Last hidden states [L, H] of one sequence."""
    H, nh = cfg.hidden, cfg.heads
    d = H // nh
    L = len(ids)
    f = lambda n: np.asarray(W[n], np.float64)
    x = f("word_emb")[ids]
    if cfg.position == 0:
        x = x + f("pos_emb")[np.minimum(np.arange(L), cfg.max_pos - 1)]
    x = x + f("type_emb")[0]
    x = layer_norm(x, f("emb_ln_g"), f("emb_ln_b"), cfg.ln_eps)
    bias = lambda n: f(n) if n in W else 0.0
    for l in range(cfg.layers):
        q = x @ f(f"q_w.{l}") + bias(f"q_b.{l}")
        k = x @ f(f"k_w.{l}") + bias(f"k_b.{l}")
        v = x @ f(f"v_w.{l}") + bias(f"v_b.{l}")
        q, k, v = (t.reshape(L, nh, d) for t in (q, k, v))
        if cfg.position == 1:
            q, k = rope_rotate(q, cfg.rope_base), rope_rotate(k, cfg.rope_base)
        s = np.einsum("qhd,khd->hqk", q, k) / np.sqrt(d)
        p = np.exp(s - s.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        ctx = np.einsum("hqk,khd->qhd", p, v).reshape(L, H)
        x = layer_norm(x + ctx @ f(f"o_w.{l}") + bias(f"o_b.{l}"), f(f"attn_ln_g.{l}"),
                       f(f"attn_ln_b.{l}"), cfg.ln_eps)
        u = x @ f(f"inter_w.{l}") + bias(f"inter_b.{l}")
        if cfg.activation == 4:
            I = cfg.intermediate
            g, up = u[:, :I], u[:, I:]
            h = g / (1.0 + np.exp(-g)) * up
        else:
            h = gelu_tanh(u)
        x = layer_norm(x + h @ f(f"out_w.{l}") + bias(f"out_b.{l}"), f(f"out_ln_g.{l}"),
                       f(f"out_ln_b.{l}"), cfg.ln_eps)
    return x


def forward(cfg, W, ids, lengths, pool):
    out, off = [], 0
    for L in lengths:
        x = encode_sequence(cfg, W, np.asarray(ids[off:off + L]))
        off += L
        if pool == 0:
            out.append(np.tanh(x[0] @ np.asarray(W["pool_w"], np.float64) + W["pool_b"]))
        else:
            p = x.mean(0)
            out.append(p / max(np.linalg.norm(p), 1e-12) if pool == 2 else p)
    return np.array(out)
