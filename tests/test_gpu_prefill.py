"""Batched prefill (vx_prefill: MFMA GEMMs over chunks of up to 256 tokens)
against the reference semantics, one backboneStep per prompt token
(src/engine.ts:2457-2472), as restated by the oracle: the KV cache of every
layer, the last token's W.normed and the position afterwards, with voice
rows spliced over [audio_start, audio_start + audio_count)."""
import os

import numpy as np
import pytest

import oracle as O
from vxtest import gpu_engine, max_rel_err, oracle_engine

pytestmark = pytest.mark.gpu

SEED = 0


def oracle_prefill(o, tokens, a_start, a_count, voice):
    for i, t in enumerate(tokens):
        if voice is not None and a_start <= i < a_start + a_count:
            o.backbone_step(int(t), 2, voice[i - a_start])
        else:
            o.backbone_step(int(t))


def check_kv(g, o, layers, npos, bar=1e-3):
    for l in range(layers):
        for w in (0, 1):
            got = g.read_kv(l, w, 0, npos)
            ref = o.kv(l, w)[:npos]
            err = max_rel_err(got, ref)
            assert err < bar, (l, w, err)


@pytest.mark.parametrize("n,a_start,a_count,layers", [(40, 5, 8, 2), (7, 0, 0, 2), (256, 2, 64, 2),
                                                    (520, 100, 218, 1)])
def test_prefill_matches_single_steps(n, a_start, a_count, layers):
    """One chunk: GEMM columns sized to the prompt (2 x n rounded up to 128)."""
    print(f"[prefill] {layers} layers, {n} tokens, voice rows {a_start}+{a_count}", flush=True)
    g = gpu_engine(n_layers=layers, max_seq=1024)
    o = oracle_engine(n_layers=layers, max_seq=1024)
    try:
        rng = np.random.default_rng(n)
        tokens = rng.integers(0, 131072, n)
        voice = O.gen_f32(SEED + n, "voice", max(a_count, 1) * 3072).reshape(-1, 3072)
        g.prefill(tokens, a_start, a_count, voice if a_count else None)
        oracle_prefill(o, tokens, a_start, a_count, voice if a_count else None)
        assert g.position == n
        check_kv(g, o, layers, n)
        assert max_rel_err(g.debug_read("normed", 3072), o.buffer("normed")) < 1e-3
        # decoding continues from the prefilled state
        _, gn = g.backbone_step(24, 1)
        o.backbone_step(24, 1)
        assert max_rel_err(gn, o.buffer("normed")) < 1e-3
    finally:
        g.destroy()
        o.close()


def test_prefill_two_chunks_after_context():
    """300 tokens on top of 10 cached positions in 256-token chunks: chunks
    of 256 and 44, the second attending to the first through the cache."""
    print("[prefill] 1 layer, 10 + 300 tokens, 256-token chunks", flush=True)
    os.environ["VX_PREFILL_CHUNK"] = "256"
    try:
        g = gpu_engine(n_layers=1, max_seq=512)
    finally:
        del os.environ["VX_PREFILL_CHUNK"]
    o = oracle_engine(n_layers=1, max_seq=512)
    try:
        rng = np.random.default_rng(7)
        head = rng.integers(0, 131072, 10)
        for t in head:
            g.backbone_step(int(t))
            o.backbone_step(int(t))
        tokens = rng.integers(0, 131072, 300)
        voice = O.gen_f32(SEED + 3, "voice", 20 * 3072).reshape(20, 3072)
        g.prefill(tokens, 250, 20, voice)  # voice rows straddle the chunk boundary
        oracle_prefill(o, tokens, 250, 20, voice)
        assert g.position == 310
        check_kv(g, o, 1, 310)
        assert max_rel_err(g.debug_read("normed", 3072), o.buffer("normed")) < 1e-3
    finally:
        g.destroy()
        o.close()


def test_prefill_argument_errors():
    import voxtral_amd as V
    g = gpu_engine(n_layers=1, max_seq=64)
    try:
        with pytest.raises(V.VoxtralError, match="out of range"):
            g.prefill([1, 2, 131072])
        with pytest.raises(V.VoxtralError, match="max_seq_len"):
            g.prefill(np.ones(65, np.int32))
        assert g.position == 0
    finally:
        g.destroy()
