"""Float64 numpy statement of the Voxtral backbone layer and FM loop, written
from the model definition (Ministral decoder layer: RMSNorm, interleaved RoPE,
GQA attention, SwiGLU; FM: 3-token bidirectional transformer, CFG, Euler,
FSQ).  It shares no code with the oracle; tests use it to pin the oracle's
arithmetic to the mathematics within float32 rounding tolerance."""
import numpy as np


def f16(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float64)


def rmsnorm(x, w, eps):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x) + eps) * w


def rope_interleaved(x, head_dim, pos, theta):
    x = np.asarray(x, np.float64).reshape(-1, head_dim).copy()
    i = np.arange(head_dim // 2)
    ang = pos * theta ** (-2.0 * i / head_dim)
    c, s = np.cos(ang), np.sin(ang)
    x0, x1 = x[:, 0::2].copy(), x[:, 1::2].copy()
    x[:, 0::2] = x0 * c - x1 * s
    x[:, 1::2] = x0 * s + x1 * c
    return x.ravel()


def gqa_decode(q, K, V, n_heads, n_kv, hd):
    """q [n_heads*hd]; K,V [seq, n_kv*hd] -> [n_heads*hd]."""
    out = np.zeros(n_heads * hd)
    rep = n_heads // n_kv
    for h in range(n_heads):
        kh = h // rep
        qh = q[h * hd:(h + 1) * hd]
        s = K[:, kh * hd:(kh + 1) * hd] @ qh / np.sqrt(hd)
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h * hd:(h + 1) * hd] = p @ V[:, kh * hd:(kh + 1) * hd]
    return out


def silu(g):
    return g / (1.0 + np.exp(-g))


def decoder_layer(x, W, pos, Kc, Vc, cfg):
    """One backbone layer at position pos.  W: dict of f64 arrays; Kc/Vc
    [max_seq, kvd] f64 caches (modified).  Returns (h_attn, h_out)."""
    hd, nh, nkv = cfg["head_dim"], cfg["n_heads"], cfg["n_kv_heads"]
    n = rmsnorm(x, W["attn_norm"], cfg["eps"])
    q = rope_interleaved(W["wq"] @ n, hd, pos, cfg["theta"])
    k = rope_interleaved(W["wk"] @ n, hd, pos, cfg["theta"])
    v = W["wv"] @ n
    Kc[pos], Vc[pos] = k, v
    a = gqa_decode(q, Kc[:pos + 1], Vc[:pos + 1], nh, nkv, hd)
    h = x + W["wo"] @ a
    n2 = rmsnorm(h, W["ffn_norm"], cfg["eps"])
    out = h + W["w2"] @ (silu(W["w1"] @ n2) * (W["w3"] @ n2))
    return h, out


def time_embedding(dim, t):
    half = dim // 2
    f = np.exp(-np.log(1e4) * np.arange(half) / half)
    return np.concatenate([np.cos(t * f), np.sin(t * f)])


def fm_layer(seq, W, cfg):
    """seq [3, dim] -> [3, dim]; bidirectional attention, no RoPE."""
    hd, nh, nkv = cfg["head_dim"], cfg["n_heads"], cfg["n_kv_heads"]
    rep = nh // nkv
    n = np.stack([rmsnorm(s, W["attn_norm"], 1e-5) for s in seq])
    q, k, v = n @ W["wq"].T, n @ W["wk"].T, n @ W["wv"].T
    a = np.zeros((3, nh * hd))
    for h in range(nh):
        kh = h // rep
        qh, kk, vv = q[:, h * hd:(h + 1) * hd], k[:, kh * hd:(kh + 1) * hd], v[:, kh * hd:(kh + 1) * hd]
        s = qh @ kk.T / np.sqrt(hd)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        a[:, h * hd:(h + 1) * hd] = p @ vv
    h1 = seq + a @ W["wo"].T
    n2 = np.stack([rmsnorm(s, W["ffn_norm"], 1e-5) for s in h1])
    return h1 + (silu(n2 @ W["w1"].T) * (n2 @ W["w3"].T)) @ W["w2"].T


def fm_forward(normed, noise, G, layers, cfg, nfe=8, alpha=1.2):
    """Returns (semantic_logits, x_final, codes)."""
    sem = G["sem_out"] @ normed
    llm = G["llm_proj"] @ normed
    x = np.asarray(noise, np.float64).copy()
    for step in range(nfe - 1):
        t, dt = step / (nfe - 1), 1.0 / (nfe - 1)
        tp = G["time_proj"] @ time_embedding(cfg["dim"], t)
        xp = G["input_proj"] @ x
        vel = []
        for cond in (llm, np.zeros_like(llm)):
            seq = np.stack([xp, tp, cond])
            for W in layers:
                seq = fm_layer(seq, W, cfg)
            vel.append(G["ac_out"] @ rmsnorm(seq[0], G["fm_norm"], 1e-5))
        v = alpha * vel[0] + (1 - alpha) * vel[1]
        x = x + v * dt
    codes = np.clip(np.round((np.clip(x, -1, 1) + 1) * 0.5 * 20), 0, 20).astype(np.uint32) + 2
    return sem, x, codes
