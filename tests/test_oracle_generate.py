"""Pins the oracle's generate() restatement (vxo_generate, restating
src/engine.ts:2416-2585) on the CPU:
  - it equals the reference's sequence of steps spelled out here with the
    oracle's individually pinned primitives: one backboneStep per prompt token
    with the voice rows spliced at [audioTokenStart, +count), the AUDIO(24)
    kick through the text embedding, frame 0 FM only, later frames' multi-
    codebook embedding, the per-position FM dataflow of the reference
    (fmForward, not the batched one vxo_generate uses), index 0 and >= 8194
    masked before the argmax, and the Box-Muller fm.noise stream at
    frame*36 + i;
  - voice rows equal to the [AUDIO] token's own embedding change nothing, so
    the splice covers exactly the audio span (shifting it by one position
    would replace the BEGIN_AUDIO or NEXT_AUDIO_TEXT embedding);
  - a semantic code <= 1 ends the loop (EOS) and teacher forcing hands the
    forced codes to the next frame.
Small dims keep it fast: 1 backbone layer, 1 FM layer, a 2048-token vocab."""
import numpy as np

import oracle as O

SEED, SEED_NOISE = 0, 11
SEM_HEAD = "acoustic_transformer.semantic_codebook_output.weight"


def small_engine():
    cfg = O.default_config(n_layers=1, fm_layers=1, vocab_size=2048)
    e = O.OracleEngine(cfg, max_seq=128)
    e.init_synthetic(SEED, 0.02)
    return e


def prompt():
    rng = np.random.default_rng(4)
    toks = [1, 25] + [24] * 6 + [36] + rng.integers(100, 2048, 9).tolist() + [35, 25]
    return toks, 2, 6


def noise(f):
    return O.gen_gauss_f32(SEED_NOISE, "fm.noise", 36 * (f + 1))[36 * f:]


def masked_argmax(logits):
    x = np.array(logits, np.float32, copy=True)
    x[0] = -np.inf
    x[8194:] = -np.inf
    return O.argmax(x)


def test_generate_is_the_reference_sequence_of_steps():
    toks, a0, na = prompt()
    voice = O.gen_f32(3, "voice.rows", na * 3072) * 0.1
    frames = 4
    e = small_engine()
    got = e.generate(toks, a0, na, voice, frames, noise_seed=SEED_NOISE, want_normed=True,
                     want_logits=True)
    pos_gen = e.position
    r = small_engine()
    r.reset()
    for i, t in enumerate(toks):  # src/engine.ts:2457-2472
        if a0 <= i < a0 + na:
            r.backbone_step(t, precomputed=voice[(i - a0) * 3072:(i - a0 + 1) * 3072])
        else:
            r.backbone_step(t)
    r.backbone_step(24)  # :2478-2487
    for f in range(frames):
        if f > 0:  # :2499-2541
            r.backbone_step_codes()
        np.testing.assert_array_equal(got["normed"][f], r.buffer("normed"))
        r.fm_forward(noise(f), batched=False)  # the reference's per-position dataflow
        np.testing.assert_array_equal(got["logits"][f], r.buffer("semantic_logits"))
        code = masked_argmax(r.buffer("semantic_logits"))  # :2556-2565
        assert int(got["semantic"][f]) == code and code > 1
        np.testing.assert_array_equal(got["acoustic"][f], r.acoustic_codes)
        np.testing.assert_array_equal(got["x_t"][f], r.buffer("x_t"))
        r.semantic_code = code  # :2573-2575
    assert got["frames"] == frames
    assert pos_gen == r.position == len(toks) + 1 + frames - 1


def test_voice_rows_equal_to_the_token_embedding_change_nothing():
    toks, a0, na = prompt()
    e = small_engine()
    emb = O.f16_bits_to_f32(e.weight("mm_audio_embeddings.tok_embeddings.weight")
                            .reshape(-1, 3072)[24])
    same = np.tile(emb, na)
    plain = e.generate(toks, a0, na, None, 2, noise_seed=SEED_NOISE, want_normed=True)
    spliced = e.generate(toks, a0, na, same, 2, noise_seed=SEED_NOISE, want_normed=True)
    np.testing.assert_array_equal(plain["normed"], spliced["normed"])
    # the same rows one position early or late do change the result
    for start in (a0 - 1, a0 + 1):
        moved = e.generate(toks, start, na, same, 1, noise_seed=SEED_NOISE, want_normed=True)
        assert not np.array_equal(moved["normed"][0], plain["normed"][0])


def test_eos_and_teacher_forcing():
    toks, a0, na = prompt()
    e = small_engine()
    free = e.generate(toks, a0, na, None, 3, noise_seed=SEED_NOISE, want_normed=True)
    assert free["frames"] == 3
    # forcing the free run's own codes reproduces it
    again = e.generate(toks, a0, na, None, 3, noise_seed=SEED_NOISE,
                       forced_semantic=free["semantic"], forced_acoustic=free["acoustic"])
    np.testing.assert_array_equal(again["semantic"], free["semantic"])
    np.testing.assert_array_equal(again["x_t"], free["x_t"])
    # forcing other codes changes the next frame's input, not the current frame
    forced_sem = np.array([7, 8, 9], np.uint32)
    forced_ac = np.full((3, 36), 12, np.uint32)
    f2 = e.generate(toks, a0, na, None, 3, noise_seed=SEED_NOISE, forced_semantic=forced_sem,
                    forced_acoustic=forced_ac, want_normed=True)
    np.testing.assert_array_equal(f2["normed"][0], free["normed"][0])
    assert not np.array_equal(f2["normed"][1], free["normed"][1])
    # a semantic-head row 1 aligned with frame 0's backbone output: EOS at
    # frame 0, before any frame is kept, and the position stays at prompt + kick
    n0 = free["normed"][0].astype(np.float64)
    W = e.weight(SEM_HEAD).reshape(8320, 3072).copy()
    W[1] = (30.0 * n0 / (n0 @ n0)).astype(np.float16).view(np.uint16)
    e.set_weight(SEM_HEAD, W)
    eos = e.generate(toks, a0, na, None, 3, noise_seed=SEED_NOISE)
    assert eos["frames"] == 0 and int(eos["semantic"][0]) == 1
    assert e.position == len(toks) + 1
    # ignore_eos keeps going; forcing frame 0 also does
    assert e.generate(toks, a0, na, None, 2, noise_seed=SEED_NOISE, ignore_eos=True)["frames"] == 2
    kept = e.generate(toks, a0, na, None, 2, noise_seed=SEED_NOISE,
                      forced_semantic=free["semantic"][:1], forced_acoustic=free["acoustic"][:1])
    assert kept["frames"] >= 1 and int(kept["semantic"][0]) == 1
