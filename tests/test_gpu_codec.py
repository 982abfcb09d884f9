"""The codec decoder on MFMA (vx_codec_decode) against the oracle's
restatement of codecDecode (src/engine.ts:1402-1713): every intermediate of
debugCodecDecode and the waveform, on the same seeded weights and codes;
chunked GEMMs; codes outside the tables; reloaded weights; generate()'s
audio; argument errors."""
import os

import numpy as np
import pytest

import oracle as O
import voxtral_amd as V
from vxtest import SEED, STD, gpu_engine, max_rel_err

pytestmark = pytest.mark.gpu

BAR = 1e-3  # f32 restatement vs f32-accurate MFMA GEMMs (measured ~1e-5)


@pytest.fixture(scope="module")
def oracle_codec():
    o = O.OracleCodec()
    o.init_synthetic(SEED, STD)
    yield o
    o.close()


@pytest.fixture(scope="module")
def engine():
    g = gpu_engine(n_layers=1, max_seq=64)
    yield g
    g.destroy()


def random_codes(T, seed):
    rng = np.random.default_rng(seed)
    return (rng.integers(2, 8194, T).astype(np.uint32),
            rng.integers(2, 23, (T, 36)).astype(np.uint32))


def check_all(g, o, sem, ac, bar=BAR):
    ref = o.decode_all(sem, ac)
    for name in V.CODEC_STOPS:
        got = g.codec_decode_to(sem, ac, name)
        assert got.shape == ref[name].shape, name
        err = max_rel_err(got, ref[name])
        assert err < bar, (name, err)


@pytest.mark.parametrize("T", [1, 4, 9])
def test_every_intermediate_matches_oracle(engine, oracle_codec, T):
    print(f"[codec] {T} frames, all intermediates", flush=True)
    sem, ac = random_codes(T, T)
    check_all(engine, oracle_codec, sem, ac)
    audio = engine.codec_decode(sem, ac)
    assert audio.shape == (T * 1920,)
    assert np.array_equal(audio, engine.codec_decode_to(sem, ac, "audio"))


def test_chunked_gemms(oracle_codec):
    """128-token GEMM chunks: 17 frames give 136 tokens in the last stage,
    so the chunk boundary falls inside the attention window and the convs'
    receptive fields."""
    print("[codec] 17 frames in 128-token chunks", flush=True)
    os.environ["VX_CODEC_CHUNK"] = "128"
    try:
        g = gpu_engine(n_layers=1, max_seq=64)
    finally:
        del os.environ["VX_CODEC_CHUNK"]
    try:
        sem, ac = random_codes(17, 17)
        ref = oracle_codec.decode_all(sem, ac)
        for name in ("after_stage2_conv_up", "after_stage3_transformer", "audio"):
            assert max_rel_err(g.codec_decode_to(sem, ac, name), ref[name]) < BAR, name
    finally:
        g.destroy()


def test_codes_outside_the_tables(engine, oracle_codec):
    """Semantic codes 8192 and 8193 (which generate() can emit) and beyond
    read a zero codebook row; acoustic codes below 2 wrap as u32."""
    print("[codec] out-of-table codes", flush=True)
    sem = np.array([8192, 8193, 0, 1, 2, 4_000_000_000], np.uint32)
    ac = np.full((6, 36), 12, np.uint32)
    ac[2, :4] = [0, 1, 22, 23]
    cat = engine.codec_decode_to(sem, ac, "concat").reshape(6, 292)
    assert not cat[[0, 1, 5], :256].any()
    assert cat[2, 256] == np.float32(np.float32(2 ** 32 - 2) * 2 / 20 - 1)
    f32 = np.float32
    assert cat[2, 258] == 1.0 and cat[2, 259] == f32(f32(21) * f32(2) / f32(20)) - f32(1)
    check_all(engine, oracle_codec, sem[[0, 1, 3, 4]], ac[[0, 1, 3, 4]])


def test_reloaded_weights_rebuild_the_operands(oracle_codec):
    """Changing a codebook usage vector and a conv gain after a decode: the
    derived operands (normalised codebook, weight-norm scales) follow."""
    print("[codec] reload after decode", flush=True)
    g = gpu_engine(n_layers=1, max_seq=64)
    o = O.OracleCodec()
    o.init_synthetic(SEED, STD)
    try:
        sem, ac = random_codes(3, 5)
        g.codec_decode(sem, ac)
        rng = np.random.default_rng(2)
        usage = (np.abs(rng.standard_normal(8192)) * 4).astype(np.float16).view(np.uint16)
        gain = (1 + rng.standard_normal(1024) * 0.3).astype(np.float16).view(np.uint16)
        for name, bits, shape in (
                ("audio_tokenizer.quantizer.semantic_codebook.cluster_usage", usage, [8192]),
                ("audio_tokenizer.decoder_blocks.4.conv.parametrizations.weight.original0", gain,
                 [1024, 1, 1])):
            g.load_tensor(name, bits, shape)
            o.set_weight(name, bits)
        check_all(g, o, sem, ac)
    finally:
        g.destroy()
        o.close()


def test_generate_returns_the_decoded_frames(engine):
    print("[codec] generate() audio", flush=True)
    r = engine.generate([1, 25, 24, 24, 35, 500, 24], 2, 2, None, 4, sampling="greedy", seed=3,
                        ignore_eos=True)
    n = r["stats"]["framesGenerated"]
    assert n == 4 and r["audio"].shape == (4 * 1920,)
    assert r["stats"]["codecMs"] > 0
    again = engine.codec_decode(r["semanticCodes"], r["acousticCodes"])
    assert np.array_equal(r["audio"], again)


def test_errors_and_codec_free_engine(engine):
    with pytest.raises(V.VoxtralError, match="bad codec arguments"):
        engine.codec_decode(np.zeros(0, np.uint32), np.zeros((0, 36), np.uint32))
    with pytest.raises(ValueError):
        engine.codec_decode([2, 3], np.zeros((3, 36), np.uint32))
    cfg = V.default_config(n_layers=1, codec=0)
    g = V.VoxtralEngine(cfg, max_seq_len=32).init()
    try:
        g.init_synthetic(SEED, STD)
        with pytest.raises(V.VoxtralError, match="without the codec"):
            g.codec_decode([2], np.full((1, 36), 12, np.uint32))
        r = g.generate([1, 24], 0, 0, None, 2, sampling="greedy", ignore_eos=True)
        assert r["stats"]["framesGenerated"] == 2 and r["audio"].size == 0
        with pytest.raises(V.VoxtralError, match="Unknown tensor"):
            g.load_tensor("audio_tokenizer.output_proj.conv.parametrizations.weight.original0",
                          np.zeros(240, np.uint16), [240, 1, 1])
    finally:
        g.destroy()
