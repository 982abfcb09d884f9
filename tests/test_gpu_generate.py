"""GPU parity of generate() (src/engine.ts:2416-2585): vx_generate against the
oracle's restatement of the same orchestration (oracle/vx_oracle.c,
vxo_generate): batched prompt prefill with the reference's real voice rows
spliced over the [AUDIO] positions, the AUDIO kick, frame 0 FM only, later
frames embedding the previous codes, the masked greedy semantic code, the
seeded fm.noise stream, and EOS on a semantic code <= 1.

Teacher forced: the oracle runs the same prompt, and after each frame it
takes the GPU's codes as the state the next frame embeds, so a frame's codes
are compared from the same inputs (a free-running comparison diverges after
the first code that sits on a rounding boundary).  Bars:
  - acoustic codes equal, except where the oracle's x_t lies within X_TOL of
    an FSQ rounding boundary (the measured GPU-oracle |dx| is about 2e-5);
  - the semantic code equal, or the GPU's pick within SEM_TOL of the
    oracle's masked maximum logit (a near tie);
  - every code identical on >= 99% of frames;
  - the same framesGenerated and the same final position.
"""
import math

import numpy as np
import pytest

import oracle as O
from vxtest import (fsq_margin, gpu_engine, max_rel_err, oracle_engine, tts_prompt,
                    voice_rows)

pytestmark = pytest.mark.gpu

X_TOL = 1e-3     # x units (codes are 0.1 apart in x)
SEM_TOL = 0.05   # logit units (GPU-oracle logit differences are about 1e-3)
SEM_HEAD = "acoustic_transformer.semantic_codebook_output.weight"
VALID = 8194


def masked(logits):
    m = np.array(logits, np.float64, copy=True)
    m[0] = -np.inf
    m[VALID:] = -np.inf
    return m


def compare(tag, gpu, ref):
    """gpu: generate() result; ref: the oracle's forced run on gpu's codes"""
    n = gpu["stats"]["framesGenerated"]
    assert len(gpu["semanticCodes"]) == n
    same = 0
    for f in range(n):
        gs, gac = gpu["semanticCodes"][f], np.array(gpu["acousticCodes"][f], np.uint32)
        os_, oac, ox = int(ref["semantic"][f]), ref["acoustic"][f], ref["x_t"][f]
        lg = masked(ref["logits"][f])
        gap = float(lg.max() - lg[gs])
        diff = gac != oac
        print(f"[{tag}] frame {f}: semantic {gs}/{os_} (gap {gap:.1e}), codes "
              f"{36 - int(diff.sum())}/36, nearest boundary {fsq_margin(ox).min():.1e}",
              flush=True)
        assert 1 < gs < VALID, (f, gs)
        assert gs == os_ or gap <= SEM_TOL, (f, gs, os_, gap)
        assert np.all(fsq_margin(ox)[diff] <= 10 * X_TOL), (f, np.nonzero(diff))
        same += int(gs == os_ and not diff.any())
    print(f"[{tag}] {same}/{n} frames with every code identical", flush=True)
    assert same >= math.ceil(0.99 * n)
    return same


def forced_oracle(o, toks, a0, na, voice, gpu, max_frames, seed, ignore_eos=False, **kw):
    n = gpu["stats"]["framesGenerated"]
    return o.generate(toks, a0, na, voice, max_frames, noise_seed=seed, ignore_eos=ignore_eos,
                      forced_semantic=np.array(gpu["semanticCodes"], np.uint32),
                      forced_acoustic=np.array(gpu["acousticCodes"], np.uint32).reshape(n, 36),
                      want_logits=True, **kw)


@pytest.mark.parametrize("layers,n_tok,n_voice,frames", [(2, 256, 64, 12), (26, 64, 32, 100)])
def test_generate_matches_oracle(layers, n_tok, n_voice, frames):
    """generate() in greedy mode, through the captured frame graphs the
    benchmark times, frame by frame against the oracle's serial run
    (src/engine.ts:2498-2585); at full depth over 100 frames, so that the
    bar of identical codes on >= 99% of frames is a count of 99."""
    print(f"[generate] {layers} layers, {n_tok}-token prompt, {n_voice} voice rows, "
          f"{frames} frames", flush=True)
    toks, a0, na = tts_prompt(n_tok, n_voice, seed=layers)
    voice = voice_rows(n_voice)
    seed = 5
    g = gpu_engine(n_layers=layers, max_seq=512)
    try:
        out = g.generate(toks, a0, na, voice, frames, sampling="greedy", seed=seed)
        gpos = g.position
    finally:
        g.destroy()
    n = out["stats"]["framesGenerated"]
    o = oracle_engine(n_layers=layers, max_seq=512)
    try:
        ref = forced_oracle(o, toks, a0, na, voice, out, frames, seed)
        # the same frame count (random weights: no EOS expected at these seeds)
        assert ref["frames"] == n == frames, (ref["frames"], n)
        assert gpos == o.position == len(toks) + 1 + (n - 1), (gpos, o.position)
        compare(f"{layers}L", out, ref)
    finally:
        o.close()


def eos_row(normed, k, low=-8.0, high=30.0):
    """A semantic-head row r (f16 bits) with r . normed[j] = low for j < k and
    high at j = k: the least-norm solution over the span of the frames'
    backbone outputs, so code 1 wins the masked argmax first at frame k."""
    N = np.asarray(normed[:k + 1], np.float64)
    t = np.full(k + 1, low)
    t[k] = high
    G = N @ N.T
    assert np.linalg.cond(G) < 1e8
    r = N.T @ np.linalg.solve(G, t)
    assert np.abs(r).max() < 1000.0
    r16 = r.astype(np.float16)
    got = N @ r16.astype(np.float64)
    assert np.all(np.abs(got - t) < 1.0), got
    return r16.view(np.uint16)


def test_generate_eos_and_position_rollback():
    """EOS (src/engine.ts:2568-2570) at a chosen frame k, in every sampling
    mode, with and without the speculative frame that generate() enqueues
    ahead; framesGenerated, the codes and the position equal the oracle's
    serial run.  The state left behind is the EOS frame's: normed, the
    device codes and the next FM pass with the device noise (frame counter
    k + 1) match the oracle, and so does a later backbone step."""
    layers, k, seed = 2, 4, 9
    toks, a0, na = tts_prompt(48, 16, seed=3)
    voice = voice_rows(16)
    g = gpu_engine(n_layers=layers, max_seq=256)
    o = oracle_engine(n_layers=layers, max_seq=256)
    try:
        base = g.generate(toks, a0, na, voice, k + 3, sampling="greedy", seed=seed,
                          ignore_eos=True)
        ref = forced_oracle(o, toks, a0, na, voice, base, k + 3, seed, ignore_eos=True,
                            want_normed=True)
        compare("eos-base", base, ref)
        row = eos_row(ref["normed"], k)
        W = g.read_tensor(SEM_HEAD, 8320 * 3072).reshape(8320, 3072).copy()
        W[1] = row
        g.load_tensor(SEM_HEAD, W)
        o.set_weight(SEM_HEAD, W)
        n_expect = len(toks) + 1 + k  # prompt, kick, steps of frames 1..k
        post = {}
        for max_frames in (k + 3, k + 1):  # speculative frame k+1 enqueued, or not
            out = g.generate(toks, a0, na, voice, max_frames, sampling="greedy", seed=seed)
            print(f"[eos] greedy, max_frames {max_frames}: {out['stats']['framesGenerated']} "
                  f"frames, position {g.position}", flush=True)
            assert out["stats"]["framesGenerated"] == k
            assert out["semanticCodes"] == base["semanticCodes"][:k]
            assert out["acousticCodes"] == base["acousticCodes"][:k]
            assert g.position == n_expect
            # the state the EOS frame left, then one FM pass from it with the
            # device noise
            normed = g.debug_read("normed", 3072)
            sem, ac = g.get_codes()
            fm_codes = g.fm_step_and_read()
            post[max_frames] = (normed, sem, ac, fm_codes, g.debug_read("x_history", 36))
        r2 = o.generate(toks, a0, na, voice, k + 3, noise_seed=seed,
                        forced_semantic=np.array(out["semanticCodes"], np.uint32),
                        forced_acoustic=np.array(out["acousticCodes"], np.uint32).reshape(k, 36),
                        want_logits=True)
        assert r2["frames"] == k and int(r2["semantic"][k]) == 1
        assert o.position == n_expect
        # frames 0..k drew noise rows 0..k; the next FM pass draws row k + 1
        noise = O.gen_gauss_f32(seed, "fm.noise", 36 * (k + 2))[36 * (k + 1):]
        o.fm_forward(noise, batched=True)
        safe = fsq_margin(o.buffer("x_t")) * 0.1 >= X_TOL  # margin in x units, as in the frame bars
        for max_frames, (normed, sem, ac, fm_codes, x0) in post.items():
            err = max_rel_err(normed, ref["normed"][k])
            print(f"[eos] max_frames {max_frames}: normed max rel err {err:.2e}, "
                  f"FM codes equal on {int(np.sum(fm_codes[safe] == o.acoustic_codes[safe]))}/"
                  f"{int(safe.sum())}", flush=True)
            assert err < 1e-3
            assert sem == 1 and list(ac) == list(base["acousticCodes"][k])
            assert np.array_equal(x0, noise)
            assert np.array_equal(fm_codes[safe], o.acoustic_codes[safe])
        # the state generate() left behind: one more step from it on both sides
        _, gn = g.backbone_step(token=7)
        o.backbone_step(token=7)
        err = max_rel_err(gn, o.buffer("normed"))
        print(f"[eos] step after generate: normed max rel err {err:.2e}", flush=True)
        assert err < 1e-3
        # EOS at frame 0, whose backbone output does not depend on the
        # sampling mode: every mode stops there, position = prompt + kick
        n0 = np.asarray(ref["normed"][0], np.float64)
        W[1] = (30.0 * n0 / (n0 @ n0)).astype(np.float16).view(np.uint16)
        g.load_tensor(SEM_HEAD, W)
        for mode in ("greedy", "top_p", "top_p_host"):
            for max_frames in (3, 1):
                out = g.generate(toks, a0, na, voice, max_frames, sampling=mode, seed=seed)
                print(f"[eos] {mode}, max_frames {max_frames}: "
                      f"{out['stats']['framesGenerated']} frames, position {g.position}",
                      flush=True)
                assert out["stats"]["framesGenerated"] == 0
                assert out["semanticCodes"] == [] and len(out["audio"]) == 0
                assert g.position == len(toks) + 1
    finally:
        g.destroy()
        o.close()
