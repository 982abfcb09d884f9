"""Float64 torch statement of the Voxtral codec decoder (codes -> waveform),
written from the architecture with torch's own operators: weight-normalised
causal Conv1d and ConvTranspose1d (torch._weight_norm, F.conv1d,
F.conv_transpose1d), RMSNorm (F.rms_norm), per-head QK RMSNorm, windowed
causal attention with ALiBi biases (F.scaled_dot_product_attention with a
float mask), layer-scaled residuals, SwiGLU.  It shares no code with the
oracle; tests use it to pin the oracle's codec arithmetic to the
mathematics within float32 rounding tolerance.

Decoder layout (the reference's src/engine.ts:700-770 and codecDecode
:1402-1713): VQ semantic embedding (codebook = embedding_sum / usage, stored
as f16) + FSQ-dequantised acoustic values -> causal conv k=3 -> 4 stages of
2 transformer layers (attention windows 2, 4, 8, 16), the first 3 followed
by a stride-2 transposed conv (k=4, output trimmed to 2T) -> causal conv
k=7 to 240 samples per step."""
import numpy as np
import torch
import torch.nn.functional as F

P = "audio_tokenizer."
WINDOWS = [2, 4, 8, 16]


def w64(bits, shape):
    return torch.from_numpy(np.asarray(bits, np.uint16).view(np.float16).astype(np.float64)).reshape(shape)


def causal_conv(x, v, g, k):
    """x [T][c_in]; v [c_out][c_in][k]; g [c_out] -> [T][c_out]"""
    w = torch._weight_norm(v, g.reshape(-1, 1, 1), 0)
    y = F.conv1d(F.pad(x.T.unsqueeze(0), (k - 1, 0)), w)
    return y[0].T


def conv_up(x, v, g, k=4, stride=2):
    """x [T][c_in]; v [c_in][c_out][k] (norm over dim 0) -> [stride*T][c_out]"""
    w = torch._weight_norm(v, g.reshape(-1, 1, 1), 0)
    y = F.conv_transpose1d(x.T.unsqueeze(0), w, stride=stride)
    return y[0, :, : stride * x.shape[0]].T


def alibi_window_mask(T, n_heads, W):
    i = torch.arange(T).reshape(-1, 1)
    j = torch.arange(T).reshape(1, -1)
    d = (i - j).to(torch.float64)
    slopes = torch.tensor([2.0 ** (-8.0 * (h + 1) / n_heads) for h in range(n_heads)], dtype=torch.float64)
    bias = -slopes.reshape(-1, 1, 1) * d
    allowed = (j <= i) & (i - j < W)
    return torch.where(allowed, bias, torch.tensor(float("-inf"), dtype=torch.float64))


def attention(q, k, v, n_heads, W):
    T = q.shape[0]
    hd = q.shape[1] // n_heads
    qh = q.reshape(T, n_heads, hd).transpose(0, 1).contiguous()
    kh = k.reshape(T, n_heads, hd).transpose(0, 1).contiguous()
    vh = v.reshape(T, n_heads, hd).transpose(0, 1).contiguous()
    o = F.scaled_dot_product_attention(qh, kh, vh, attn_mask=alibi_window_mask(T, n_heads, W))
    return o.transpose(0, 1).reshape(T, n_heads * hd)


def qk_norm(x, w, n_heads, eps):
    T = x.shape[0]
    hd = x.shape[1] // n_heads
    y = F.rms_norm(x.reshape(T, n_heads, hd), (hd,), eps=eps)
    return (y * w.reshape(n_heads, hd)).reshape(T, -1)


def decode(weights, semantic, acoustic, eps=0.01, qk_eps=1e-6, n_heads=8):
    """weights: name -> f16 bits (numpy).  Returns the intermediates of
    debugCodecDecode by name, float64 numpy."""
    W = lambda name, shape: w64(weights[P + name], shape)
    T = len(semantic)
    out = {}
    emb_sum = W("quantizer.semantic_codebook.embedding_sum", (8192, 256))
    usage = W("quantizer.semantic_codebook.cluster_usage", (8192,))
    cb = (emb_sum / torch.clamp(usage, min=1e-5).reshape(-1, 1)).to(torch.float16).to(torch.float64)
    sem = torch.as_tensor(np.asarray(semantic, np.int64))
    semf = torch.zeros(T, 256, dtype=torch.float64)
    ok = sem < 8192
    semf[ok] = cb[sem[ok]]
    ac = torch.as_tensor(np.asarray(acoustic, np.float64)).reshape(T, 36)
    acf = (ac - 2.0) * 2.0 / 20.0 - 1.0
    x = torch.cat([semf, acf], 1)
    out["concat"] = x
    x = causal_conv(x, W("decoder_blocks.0.conv.parametrizations.weight.original1", (1024, 292, 3)),
                    W("decoder_blocks.0.conv.parametrizations.weight.original0", (1024,)), 3)
    out["after_input_conv"] = x
    for s in range(4):
        for l in range(2):
            p = f"decoder_blocks.{1 + 2 * s}.layers.{l}."
            h = F.rms_norm(x, (1024,), W(p + "attention_norm.weight", (1024,)), eps)
            q = qk_norm(h @ W(p + "attention.wq.weight", (1024, 1024)).T, W(p + "attention.q_norm.weight", (1024,)),
                        n_heads, qk_eps)
            k = qk_norm(h @ W(p + "attention.wk.weight", (1024, 1024)).T, W(p + "attention.k_norm.weight", (1024,)),
                        n_heads, qk_eps)
            v = h @ W(p + "attention.wv.weight", (1024, 1024)).T
            a = attention(q, k, v, n_heads, WINDOWS[s])
            x = x + (a @ W(p + "attention.wo.weight", (1024, 1024)).T) * W(p + "attention_scale", (1024,))
            h = F.rms_norm(x, (1024,), W(p + "ffn_norm.weight", (1024,)), eps)
            f = F.silu(h @ W(p + "feed_forward.w1.weight", (4096, 1024)).T) * (
                h @ W(p + "feed_forward.w3.weight", (4096, 1024)).T)
            x = x + (f @ W(p + "feed_forward.w2.weight", (1024, 4096)).T) * W(p + "ffn_scale", (1024,))
        out[f"after_stage{s}_transformer"] = x
        if s < 3:
            b = f"decoder_blocks.{2 + 2 * s}.conv.parametrizations.weight."
            x = conv_up(x, W(b + "original1", (1024, 1024, 4)), W(b + "original0", (1024,)))
            out[f"after_stage{s}_conv_up"] = x
    out["audio"] = causal_conv(x, W("output_proj.conv.parametrizations.weight.original1", (240, 1024, 7)),
                               W("output_proj.conv.parametrizations.weight.original0", (240,)), 7)
    return {k: v.numpy() for k, v in out.items()}
