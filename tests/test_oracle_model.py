"""Pins the oracle's orchestration (backboneStep, fmForward) against the
float64 model in oracle_np.py on a reduced configuration."""
import numpy as np
import pytest

import oracle as O
import oracle_np as R

SMALL = dict(dim=256, n_layers=2, head_dim=64, hidden_dim=512, n_heads=4, n_kv_heads=2,
             vocab_size=512, fm_layers=2)


@pytest.fixture(scope="module")
def small():
    cfg = O.default_config(**SMALL)
    e = O.OracleEngine(cfg, max_seq=64)
    e.init_synthetic(seed=3, std=0.05)
    return e


def layer_weights(e, prefix):
    g = lambda n: R.f16(e.weight(f"{prefix}.{n}"))
    c = e.cfg
    d, qd, kvd, hd = c.dim, c.n_heads * c.head_dim, c.n_kv_heads * c.head_dim, c.hidden_dim
    return dict(attn_norm=g("attention_norm.weight"), ffn_norm=g("ffn_norm.weight"),
                wq=g("attention.wq.weight").reshape(qd, d), wk=g("attention.wk.weight").reshape(kvd, d),
                wv=g("attention.wv.weight").reshape(kvd, d), wo=g("attention.wo.weight").reshape(d, qd),
                w1=g("feed_forward.w1.weight").reshape(hd, d), w2=g("feed_forward.w2.weight").reshape(d, hd),
                w3=g("feed_forward.w3.weight").reshape(hd, d))


def test_backbone_steps_match_float64_model(small):
    e = small
    c = e.cfg
    e.reset()
    cfgd = dict(head_dim=c.head_dim, n_heads=c.n_heads, n_kv_heads=c.n_kv_heads, eps=1e-5, theta=1e6)
    Ws = [layer_weights(e, f"layers.{i}") for i in range(c.n_layers)]
    kvd = c.n_kv_heads * c.head_dim
    Kc = [np.zeros((64, kvd)) for _ in range(c.n_layers)]
    Vc = [np.zeros((64, kvd)) for _ in range(c.n_layers)]
    tok = R.f16(e.weight("mm_audio_embeddings.tok_embeddings.weight")).reshape(c.vocab_size, c.dim)
    audio = R.f16(e.weight("mm_audio_embeddings.audio_codebook_embeddings.embeddings.weight")).reshape(-1, c.dim)
    fnorm = R.f16(e.weight("norm.weight"))
    voice = np.random.RandomState(0).randn(c.dim).astype(np.float32)
    steps = [(5, 0, None), (77, 1, None), (0, 2, voice), (300, 0, None), (12, 0, None), (1, 1, None)]
    for pos, (t, mode, pre) in enumerate(steps):
        lo = e.backbone_step(t, mode, pre, lm_head=True, layer_out=True)
        x = pre.astype(np.float64) if pre is not None else (audio[t] if mode == 1 else tok[t])
        for i, W in enumerate(Ws):
            h, x = R.decoder_layer(x, W, pos, Kc[i], Vc[i], cfgd)
            s = np.abs(x).max()
            assert np.max(np.abs(lo[i, 0] - h)) <= 2e-5 * s, (pos, i)
            assert np.max(np.abs(lo[i, 1] - x)) <= 2e-5 * s, (pos, i)
        normed = R.rmsnorm(x, fnorm, 1e-5)
        np.testing.assert_allclose(e.buffer("normed"), normed, atol=2e-5 * np.abs(normed).max())
        logits = tok @ normed
        np.testing.assert_allclose(e.buffer("logits"), logits, atol=2e-5 * np.abs(logits).max())
        assert e.argmax_result == int(np.argmax(e.buffer("logits")))
        # the K cache row holds the roped key of this position
        np.testing.assert_allclose(e.kv(0, 0)[pos], Kc[0][pos], atol=2e-5 * np.abs(Kc[0][pos]).max())
    assert e.position == len(steps)


def test_layer_by_layer_read_points(small):
    """debugBackboneLayerByLayer's read points: the embedding, each layer's
    two RMSNorm outputs (attention and FFN inputs, with their gains) and
    the hidden state after each residual, against the float64 model; the
    step itself leaves the same state as a plain step."""
    e = small
    c = e.cfg
    cfgd = dict(head_dim=c.head_dim, n_heads=c.n_heads, n_kv_heads=c.n_kv_heads, eps=1e-5, theta=1e6)
    Ws = [layer_weights(e, f"layers.{i}") for i in range(c.n_layers)]
    tok = R.f16(e.weight("mm_audio_embeddings.tok_embeddings.weight")).reshape(c.vocab_size, c.dim)
    kvd = c.n_kv_heads * c.head_dim
    e.reset()
    e.backbone_step(41)
    e.backbone_step(7)
    plain = e.backbone_step(300, layer_out=True)
    normed_plain = e.buffer("normed").copy()
    e.reset()
    e.backbone_step(41)
    e.backbone_step(7)
    res = e.backbone_layer_by_layer(300)
    assert e.position == 3
    assert np.array_equal(res["final_norm"], normed_plain)
    assert np.array_equal(res["hidden"], plain[-1, 1])
    assert np.array_equal(res["embed"], tok[300].astype(np.float32))
    Kc = [np.zeros((64, kvd)) for _ in range(c.n_layers)]
    Vc = [np.zeros((64, kvd)) for _ in range(c.n_layers)]
    for pos, t in enumerate((41, 7, 300)):
        x = tok[t]
        for i, W in enumerate(Ws):
            n1 = R.rmsnorm(x, W["attn_norm"], 1e-5)
            h, x2 = R.decoder_layer(x, W, pos, Kc[i], Vc[i], cfgd)
            n2 = R.rmsnorm(h, W["ffn_norm"], 1e-5)
            if pos == 2:
                L = res["layers"][i]
                assert np.array_equal(L["attn_out"], plain[i, 0])
                assert np.array_equal(L["ffn_out"], plain[i, 1])
                for name, ref in (("attn_norm", n1), ("attn_out", h), ("ffn_norm", n2), ("ffn_out", x2)):
                    assert np.max(np.abs(L[name] - ref)) <= 2e-5 * np.abs(ref).max(), (i, name)
                # the norm outputs are not the hidden states (a swapped read point fails here)
                assert np.max(np.abs(L["attn_norm"] - h)) > 1e-3 * np.abs(h).max()
            x = x2


def test_multi_codebook_step_uses_codes(small):
    e = small
    c = e.cfg
    e.reset()
    e.semantic_code = 4000
    codes = np.arange(36, dtype=np.uint32) % 21 + 2
    e.acoustic_codes = codes
    e.backbone_step_codes()
    h1 = e.buffer("normed").copy()
    audio = O.f16_bits_to_f32(e.weight("mm_audio_embeddings.audio_codebook_embeddings.embeddings.weight")).reshape(-1, c.dim)
    emb = O.multi_codebook_embed(e.weight("mm_audio_embeddings.audio_codebook_embeddings.embeddings.weight").reshape(-1, c.dim),
                                 4000, codes, c.dim)
    e.reset()
    e.backbone_step(precomputed=emb)
    assert np.array_equal(e.buffer("normed"), h1)
    assert audio.shape[0] == 9088


@pytest.mark.parametrize("batched", [False, True])
def test_fm_forward_matches_float64_model(small, batched):
    e = small
    c = e.cfg
    e.reset()
    e.backbone_step(9)
    normed = e.buffer("normed").astype(np.float64).copy()
    noise = O.gen_f32(11, "noise", 36)
    e.fm_forward(noise, batched=batched)
    g = lambda n: R.f16(e.weight(f"acoustic_transformer.{n}"))
    d = c.dim
    G = dict(sem_out=g("semantic_codebook_output.weight").reshape(-1, d),
             llm_proj=g("llm_projection.weight").reshape(d, d),
             time_proj=g("time_projection.weight").reshape(d, d),
             input_proj=g("input_projection.weight").reshape(d, 36),
             ac_out=g("acoustic_codebook_output.weight").reshape(36, d),
             fm_norm=g("norm.weight"))
    layers = [layer_weights(e, f"acoustic_transformer.layers.{i}") for i in range(c.fm_layers)]
    cfgd = dict(dim=d, head_dim=c.head_dim, n_heads=c.n_heads, n_kv_heads=c.n_kv_heads)
    sem, x, codes = R.fm_forward(normed, noise, G, layers, cfgd)
    np.testing.assert_allclose(e.buffer("semantic_logits"), sem, atol=2e-5 * np.abs(sem).max())
    np.testing.assert_allclose(e.buffer("x_t"), x, atol=5e-5 * max(1.0, np.abs(x).max()))
    # codes agree wherever x is not within 1e-4 of an FSQ decision boundary
    u = (np.clip(x, -1, 1) + 1) * 10
    safe = np.abs(u - np.floor(u) - 0.5) > 1e-3
    assert np.array_equal(e.acoustic_codes[safe], codes[safe])
    assert e.semantic_code == int(np.argmax(e.buffer("semantic_logits")))


def test_fm_batched_dataflow_is_bit_identical(small):
    e = small
    e.reset()
    e.backbone_step(17)
    noise = O.gen_f32(5, "noise", 36)
    e.fm_forward(noise)
    a = (e.buffer("x_t").copy(), e.buffer("semantic_logits").copy(), e.acoustic_codes)
    e.fm_forward(noise, batched=True)
    assert np.array_equal(a[0], e.buffer("x_t"))
    assert np.array_equal(a[1], e.buffer("semantic_logits"))
    assert np.array_equal(a[2], e.acoustic_codes)
