"""Shared helpers of the parity tests: the comparison functions and engine
pairs (HIP engine + CPU oracle) built from the same seeded synthetic data."""
import numpy as np

import oracle as O

SEED = 0
STD = 0.02


def max_rel_err(actual, expected):
    """max |a-e| / max(|e|, 1e-2*||e||_inf): the hidden-state tolerance
    metric (bound 1e-2 for f16 weights with f32 accumulation)."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    floor = 1e-2 * max(np.abs(e).max(), 1e-30)
    return float(np.max(np.abs(a - e) / np.maximum(np.abs(e), floor)))


def ref_allclose(actual, expected, atol=0.01, rtol=0.01):
    """allclose of the reference test utilities (src/npy.ts:122-169):
    passes when |a-e| <= atol + rtol*|e| everywhere."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    return bool(np.all(np.abs(a - e) <= atol + rtol * np.abs(e)))


def oracle_engine(n_layers=1, fm_layers=3, max_seq=1024, seed=SEED, std=STD):
    cfg = O.default_config(n_layers=n_layers, fm_layers=fm_layers)
    e = O.OracleEngine(cfg, max_seq=max_seq)
    e.init_synthetic(seed, std)
    return e


def gpu_engine(n_layers=1, fm_layers=3, max_seq=1024, seed=SEED, std=STD, kv_f16=False):
    import voxtral_amd as V
    cfg = V.default_config(n_layers=n_layers, fm_layers=fm_layers, kv_f16=int(kv_f16))
    g = V.VoxtralEngine(cfg, max_seq_len=max_seq).init()
    g.init_synthetic(seed, std)
    return g


def fill_oracle_kv(o, seed, npos):
    """Same synthetic KV rows as vx_fill_kv_synthetic: f16 N(0,1) from the
    generator stream kv.<layer>.k / .v, held as f32 by the oracle."""
    kvd = o.cfg.n_kv_heads * o.cfg.head_dim
    for l in range(o.cfg.n_layers):
        for w, nm in ((0, "k"), (1, "v")):
            bits = O.gen_f16(seed, f"kv.{l}.{nm}", npos * kvd)
            o.kv(l, w)[:npos] = O.f16_bits_to_f32(bits).reshape(npos, kvd)


def masked_tree_argmax(logits):
    """Greedy semantic code: index 0 and >= 8194 masked (src/engine.ts:
    2556-2563), then the 256-lane tree argmax."""
    x = np.array(logits, np.float32, copy=True)
    x[0] = -np.inf
    x[8194:] = -np.inf
    return O.argmax(x)


VOICE_ROWS = __import__("os").path.join(__import__("os").path.dirname(__file__), "golden",
                                        "ar_male_voice_rows64.f32")


def voice_rows(n=64):
    """The reference's real voice embedding rows (ar_male, f32 [n][3072]),
    from the committed slice (tests/golden/make_voice_rows.py)."""
    a = np.fromfile(VOICE_ROWS, dtype="<f4").reshape(-1, 3072)
    assert n <= a.shape[0]
    return a[:n].copy()


def tts_prompt(n_tokens=256, n_voice=64, seed=0):
    """A prompt laid out as buildTTSPrompt does (src/tokenizer.ts:130-165):
    BOS [BEGIN_AUDIO] [AUDIO] x n_voice [NEXT_AUDIO_TEXT] text
    [REPEAT_AUDIO_TEXT] [BEGIN_AUDIO], with the text ids drawn uniformly
    from the non-special vocabulary.  Returns (tokens, audio_start, count)."""
    n_text = n_tokens - n_voice - 5
    assert n_text >= 0
    rng = np.random.default_rng(seed)
    text = rng.integers(1000, 131072, n_text).tolist()
    toks = [1, 25] + [24] * n_voice + [36] + text + [35, 25]
    return toks, 2, n_voice


def fsq_margin(x):
    """distance of x from the nearest FSQ rounding boundary, in code units
    (codes are round((clip(x)+1)/2*20)+2, boundaries at half-integers)"""
    u = (np.clip(np.asarray(x, np.float64), -1, 1) + 1) * 10
    return np.abs(u - np.floor(u) - 0.5)
