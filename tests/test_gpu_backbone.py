"""GPU parity of the backbone decode step: HIP engine (through the C ABI)
against the CPU oracle on identical seeded inputs.

Tolerance (hidden states, f16 weights with f32 accumulation): max relative
error <= 1e-2 with denominator floor 1e-2*||e||_inf, and the reference's
allclose(atol=1e-2, rtol=1e-2).  Intermediate buffers get a tighter bar:
with the default f32 KV cache they differ from the oracle only by
summation order and the f32 rounding of the rope angle.  The optional f16
KV cache is checked against the oracle's f16-KV mode."""
import numpy as np
import pytest

import oracle as O
from vxtest import (fill_oracle_kv, gpu_engine, max_rel_err, oracle_engine, ref_allclose)

pytestmark = pytest.mark.gpu

SEED = 0


@pytest.fixture(scope="module")
def pair1():
    """Single decoder layer (the 1-layer decode-at-128 workload) + full FM."""
    print("[pair1] building 1-layer engines", flush=True)
    g = gpu_engine(n_layers=1, max_seq=1024)
    o = oracle_engine(n_layers=1, max_seq=1024)
    yield g, o
    g.destroy()
    o.close()


def test_kv_generator_bit_identical(pair1):
    g, o = pair1
    g.fill_kv_synthetic(SEED, 128)
    got = g.read_kv(0, 0, 0, 128)
    ref = O.f16_bits_to_f32(O.gen_f16(SEED, "kv.0.k", 128 * 1024)).reshape(128, 1024)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    got = g.read_kv(0, 1, 100, 28)
    ref = O.f16_bits_to_f32(O.gen_f16(SEED, "kv.0.v", 128 * 1024)).reshape(128, 1024)[100:]
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    # write/read round trip of arbitrary f32 rows
    rows = O.gen_f32(SEED + 5, "kv.rows", 3 * 1024).reshape(3, 1024)
    g.write_kv(0, 1, 500, rows)
    assert np.array_equal(g.read_kv(0, 1, 500, 3), rows)


@pytest.mark.parametrize("name", ["layers.0.attention.wq.weight", "layers.0.attention.wv.weight",
                                  "layers.0.ffn_norm.weight", "layers.0.feed_forward.w2.weight",
                                  "acoustic_transformer.input_projection.weight",
                                  "mm_audio_embeddings.audio_codebook_embeddings.embeddings.weight"])
def test_weight_generator_bit_identical(pair1, name):
    """Device-side synthetic weights equal the CPU generator's bit for bit,
    f16 subnormals included."""
    g, o = pair1
    ref = o.weight(name)
    got = g.read_tensor(name, ref.size)
    assert np.array_equal(got, ref), int((got != ref).sum())


def test_load_tensor_roundtrip_and_errors(pair1):
    import voxtral_amd as V
    g, o = pair1
    name = "layers.0.attention.wk.weight"
    ref = o.weight(name).reshape(1024, 3072)
    g.load_tensor(name, ref)
    assert np.array_equal(g.read_tensor(name, ref.size), ref.ravel())
    with pytest.raises(V.VoxtralError, match="Unknown tensor"):
        g.load_tensor("layers.0.attention.wz.weight", ref)
    with pytest.raises(V.VoxtralError, match="shape mismatch"):
        g.load_tensor(name, ref.reshape(3072, 1024))
    assert g.is_ready


def test_code_and_position_argument_errors(pair1):
    """Out-of-range codes and positions are rejected on the host, before any
    kernel could index past the embedding table or the KV cache (semantic
    codes of 2^31 and more included: the bound is an unsigned compare)."""
    import voxtral_amd as V
    g, _ = pair1
    for bad in (9088, 2**31, 2**32 - 1):
        with pytest.raises(V.VoxtralError, match="semantic code"):
            g.set_semantic_code(bad)
    g.set_semantic_code(9087)  # the table's last row
    with pytest.raises(V.VoxtralError, match="acoustic code"):
        g.set_acoustic_codes(np.full(36, 23, np.uint32))
    with pytest.raises(V.VoxtralError, match="out of range"):
        g.position = 1025
    with pytest.raises(V.VoxtralError, match="out of range"):
        g.position = -1
    g.position = 1024
    with pytest.raises(V.VoxtralError, match="max_seq_len"):
        g.backbone_step(token=1)
    g.position = 0
    # KV row ranges whose end overflows int32 (checked in 64 bits)
    big = 2**31 - 8
    with pytest.raises(V.VoxtralError, match="KV range"):
        g.read_kv(0, 0, big, 16)
    with pytest.raises(V.VoxtralError, match="KV range"):
        g.write_kv(0, 0, big, np.zeros((16, 1024), np.float32))
    # voice ranges whose end overflows int32
    with pytest.raises(V.VoxtralError, match="bad prefill arguments"):
        g.prefill([1, 2, 3], audio_token_start=big, audio_token_count=64,
                  voice_embeddings=np.zeros((64, 3072), np.float32))
    with pytest.raises(V.VoxtralError, match="voice range"):
        g.generate([1, 2, 3], big, 64, np.zeros((64, 3072), np.float32), 1)
    # sampling options that would make NaN probabilities
    for bad in (dict(temperature=0.0), dict(temperature=float("nan")), dict(top_p=0.0),
                dict(top_p=float("nan")), dict(top_p=1.5), dict(temperature=float("inf"))):
        with pytest.raises(V.VoxtralError, match="top-p sampling needs"):
            g.generate([1, 2, 3], 0, 0, None, 1, sampling="top_p", **bad)
    assert g.position == 0


def test_single_layer_decode_at_128(pair1):
    g, o = pair1
    x = O.gen_f32(SEED, "input.hidden", 3072)
    g.fill_kv_synthetic(SEED, 128)
    fill_oracle_kv(o, SEED, 128)
    g.position = 128
    o.position = 128
    res = g.debug_backbone_layer_by_layer(0, precomputed=x)
    oref = o.backbone_layer_by_layer(precomputed=x)
    assert g.position == 129 and o.position == 129
    # per-kernel intermediates
    q_err = max_rel_err(g.debug_read("q", 4096), o.buffer("q"))
    a_err = max_rel_err(g.debug_read("attn_out", 4096), o.buffer("attn_out"))
    s_err = max_rel_err(g.debug_read("gate", 9216), o.buffer("gate"))
    print(f"q {q_err:.2e} attn {a_err:.2e} swiglu {s_err:.2e}")
    # q differs from the oracle by the f32 rounding of the rope angle
    # pos*freq (~|q| * pos * 2^-24 absolute) and summation order.  Real
    # defects show errors of order 1.
    assert q_err < 1e-3 and a_err < 1e-3 and s_err < 1e-3
    # the new K/V row (rope'd k, v) in the f32 cache
    for w in (0, 1):
        new = g.read_kv(0, w, 128, 1)[0]
        ref = o.kv(0, w)[128]
        np.testing.assert_allclose(new, ref, rtol=1e-3, atol=1e-4 * np.abs(ref).max())
    # every read point of debugBackboneLayerByLayer (the embedding row is
    # the precomputed input, copied)
    assert np.array_equal(res["embed"], oref["embed"])
    for name in ("attn_norm", "attn_out", "ffn_norm", "ffn_out"):
        err = max_rel_err(res["layers"][0][name], oref["layers"][0][name])
        print(f"{name} max rel err {err:.2e}")
        assert err < 2e-3
        assert ref_allclose(res["layers"][0][name], oref["layers"][0][name])
    assert np.array_equal(res["hidden"], res["layers"][0]["ffn_out"])
    err = max_rel_err(res["final_norm"], o.buffer("normed"))
    assert err < 2e-3 and ref_allclose(res["final_norm"], o.buffer("normed"))


@pytest.mark.parametrize("pos", [1, 16, 128, 512])
def test_against_reference_f32_kv(pair1, pos):
    """The spec bar against the oracle: max relative error <= 1e-2 and
    allclose(1e-2, 1e-2)."""
    g, o = pair1
    x = O.gen_f32(SEED + 7, "input.hidden", 3072)
    g.fill_kv_synthetic(SEED, pos)
    fill_oracle_kv(o, SEED, pos)
    g.position = pos
    o.position = pos
    _, gn = g.backbone_step(precomputed=x)
    o.backbone_step(precomputed=x)
    err = max_rel_err(gn, o.buffer("normed"))
    print(f"pos {pos}: vs oracle {err:.2e}")
    assert err < 1e-3 and ref_allclose(gn, o.buffer("normed"))


def test_step_matches_per_layer_path(pair1):
    """The captured decode-step graph against the per-kernel debug path on
    the same state: identical kernels, so identical results."""
    g, o = pair1
    x = O.gen_f32(SEED + 1, "input.hidden", 3072)
    g.fill_kv_synthetic(SEED, 300)
    g.position = 300
    eager = g.debug_backbone_layer_by_layer(0, precomputed=x)["final_norm"]
    g.position = 300
    _, step = g.backbone_step(precomputed=x)
    assert max_rel_err(step, eager) < 1e-6


def test_layer_read_points_agree_between_entry_points(pair1):
    """vx_backbone_step_layers (the two residual read points) and
    vx_debug_backbone_layers run the same kernels on the same state, so
    their shared read points are identical."""
    g, _ = pair1
    x = O.gen_f32(SEED + 2, "input.hidden", 3072)
    g.fill_kv_synthetic(SEED, 77)
    g.position = 77
    full = g.debug_backbone_layer_by_layer(0, precomputed=x)
    g.position = 77
    two = g.backbone_step_layers(0, precomputed=x)
    assert g.position == 78
    assert np.array_equal(two[0, 0], full["layers"][0]["attn_out"])
    assert np.array_equal(two[0, 1], full["layers"][0]["ffn_out"])


def test_eager_path_matches_graph(pair1, monkeypatch):
    """VX_NO_GRAPH=1 enqueues the step's kernels directly instead of
    replaying the captured graph (the mode kernel tracers use); both agree
    with the oracle on a 26-position context."""
    import voxtral_amd as V
    g, o = pair1
    monkeypatch.setenv("VX_NO_GRAPH", "1")
    gf = V.VoxtralEngine(V.default_config(n_layers=1), max_seq_len=64).init()
    monkeypatch.delenv("VX_NO_GRAPH")
    try:
        gf.init_synthetic(SEED, 0.02)
        x = O.gen_f32(SEED + 3, "input.hidden", 3072)
        for e in (gf, g):
            e.fill_kv_synthetic(SEED, 26)
            e.position = 26
        fill_oracle_kv(o, SEED, 26)
        o.position = 26
        _, a = gf.backbone_step(precomputed=x)
        _, b = g.backbone_step(precomputed=x)
        o.backbone_step(precomputed=x)
        assert max_rel_err(a, o.buffer("normed")) < 2e-3
        assert max_rel_err(b, o.buffer("normed")) < 2e-3
        assert max_rel_err(a, b) < 1e-6
    finally:
        gf.destroy()


@pytest.mark.parametrize("pos", [0, 1, 63, 64, 65, 511, 1023])
def test_attention_positions(pair1, pos):
    """Key counts around the split/chunk boundaries, down to a single key."""
    g, o = pair1
    x = O.gen_f32(SEED + pos, "input.hidden", 3072)
    g.fill_kv_synthetic(SEED, pos)
    fill_oracle_kv(o, SEED, pos)
    g.position = pos
    o.position = pos
    _, normed = g.backbone_step(precomputed=x)
    o.backbone_step(precomputed=x)
    a_err = max_rel_err(g.debug_read("attn_out", 4096), o.buffer("attn_out"))
    assert a_err < 1e-3, a_err
    assert max_rel_err(normed, o.buffer("normed")) < 1e-3


def test_lm_head_argmax(pair1):
    g, o = pair1
    g.reset()
    o.reset()
    for t in (1, 24, 131071):
        am = g.backbone_step_and_read(t)
        o.backbone_step(t, lm_head=True)
        lg = g.debug_read("logits", 131072)
        assert max_rel_err(lg, o.buffer("logits")) < 1e-2
        top2 = np.sort(o.buffer("logits"))[-2:]
        if top2[1] - top2[0] > 1e-3 * abs(top2[1]):
            assert am == o.argmax_result


def test_prefill_sequence_all_embedding_modes(pair1):
    g, o = pair1
    g.reset()
    o.reset()
    voice = O.gen_f32(SEED, "voice", 2 * 3072).reshape(2, 3072)
    steps = [(1, 0, None), (25, 0, None), (24, 0, voice[0]), (24, 0, voice[1]), (1000, 1, None),
             (35, 0, None)]
    for t, mode, pre in steps:
        _, gn = g.backbone_step(t, mode, pre)
        o.backbone_step(t, mode, pre)
        assert max_rel_err(gn, o.buffer("normed")) < 2e-3


@pytest.fixture(scope="module")
def pair26():
    print("[pair26] building 26-layer engines", flush=True)
    g = gpu_engine(n_layers=26, max_seq=1024)
    o = oracle_engine(n_layers=26, max_seq=1024)
    yield g, o
    g.destroy()
    o.close()


def test_full_backbone_decode_at_512(pair26):
    """26 layers, 512 cached positions, decode at position 512."""
    g, o = pair26
    x = O.gen_f32(SEED, "input.hidden", 3072)
    g.fill_kv_synthetic(SEED, 512)
    fill_oracle_kv(o, SEED, 512)
    g.position = 512
    o.position = 512
    _, gn = g.backbone_step(precomputed=x)
    o.backbone_step(precomputed=x)
    err = max_rel_err(gn, o.buffer("normed"))
    print(f"26-layer normed max rel err {err:.2e}")
    assert err < 1e-2 and ref_allclose(gn, o.buffer("normed"))
    assert max_rel_err(g.debug_read("hidden", 3072), o.buffer("hidden")) < 1e-2


def test_decode_at_512_after_real_prefill(pair26):
    """The headline workload as the benchmark builds it: a 512-token prefix of
    ids drawn uniformly from the 131072-token vocabulary (seed 0) prefilled
    with the batched GEMM prefill, then a decode step at position 512 (513
    keys) through all 26 layers.  The oracle runs the reference's per-token
    prefill (src/engine.ts:2457-2472) and the same step.  Checked: normed,
    the residual stream, and the K/V rows of layers 0, 12 and 25."""
    g, o = pair26
    g.reset()
    o.reset()
    toks = np.random.default_rng(0).integers(0, 131072, 512)
    g.prefill(toks)
    for t in toks:
        o.backbone_step(int(t))
    assert g.position == o.position == 512
    x = O.gen_f32(SEED, "input.hidden", 3072)
    _, gn = g.backbone_step(precomputed=x)
    o.backbone_step(precomputed=x)
    err = max_rel_err(gn, o.buffer("normed"))
    herr = max_rel_err(g.debug_read("hidden", 3072), o.buffer("hidden"))
    print(f"[c1] decode at 512 after a real prefill: normed {err:.2e}, hidden {herr:.2e}", flush=True)
    assert err < 1e-2 and ref_allclose(gn, o.buffer("normed"))
    assert herr < 1e-2
    for l in (0, 12, 25):
        for w in (0, 1):
            kerr = max_rel_err(g.read_kv(l, w, 0, 513), o.kv(l, w)[:513])
            print(f"[c1] layer {l} {'KV'[w]} rows 0..512: {kerr:.2e}", flush=True)
            assert kerr < 1e-2, (l, w, kerr)


def test_full_backbone_real_prefill(pair26):
    """Prompt tokens through all 26 layers from position 0 (real KV)."""
    g, o = pair26
    g.reset()
    o.reset()
    toks = [1, 25, 24, 24, 35, 500, 131000, 3]
    for t in toks:
        _, gn = g.backbone_step(t)
        o.backbone_step(t)
        err = max_rel_err(gn, o.buffer("normed"))
        assert err < 1e-2, (t, err)
    kv_g = g.read_kv(25, 0, 0, len(toks))
    kv_o = o.kv(25, 0)[:len(toks)]
    assert max_rel_err(kv_g, kv_o) < 1e-2


# ------------------------------------------------------- f16 KV cache option
@pytest.fixture(scope="module")
def pair1_f16():
    print("[pair1_f16] building 1-layer engines, f16 KV", flush=True)
    g = gpu_engine(n_layers=1, max_seq=1024, kv_f16=True)
    o = oracle_engine(n_layers=1, max_seq=1024)
    o.set_kv_f16(True)  # the oracle rounds new K/V rows to f16 as the engine stores them
    yield g, o
    g.destroy()
    o.close()


@pytest.mark.parametrize("pos", [0, 1, 65, 128, 1023])
def test_f16_kv_cache(pair1_f16, pos):
    """f16 cache: same arithmetic as the oracle's f16-KV mode; the new row
    is the f16 rounding of the oracle's f32 row."""
    g, o = pair1_f16
    x = O.gen_f32(SEED + 11 + pos, "input.hidden", 3072)
    g.fill_kv_synthetic(SEED, pos)
    fill_oracle_kv(o, SEED, pos)
    if pos:
        assert np.array_equal(g.read_kv(0, 0, 0, pos), o.kv(0, 0)[:pos])
    g.position = pos
    o.position = pos
    _, gn = g.backbone_step(precomputed=x)
    o.backbone_step(precomputed=x)
    # a K/V element whose f32 value sits near an f16 rounding boundary can
    # round the other way (one f16 ulp, 2^-11 relative)
    a_err = max_rel_err(g.debug_read("attn_out", 4096), o.buffer("attn_out"))
    assert a_err < 1e-2, a_err
    assert max_rel_err(gn, o.buffer("normed")) < 2e-3
    for w in (0, 1):
        new, ref = g.read_kv(0, w, pos, 1)[0], o.kv(0, w)[pos]
        np.testing.assert_allclose(new, ref, rtol=2e-3, atol=1e-3 * np.abs(ref).max())
    rows = O.gen_f32(SEED + 5, "kv.rows", 2 * 1024).reshape(2, 1024)
    g.write_kv(0, 1, 1000, rows)
    assert np.array_equal(g.read_kv(0, 1, 1000, 2), rows.astype(np.float16).astype(np.float32))


@pytest.mark.parametrize("kv_f16", [False, True])
def test_long_context_decode(kv_f16):
    """Consecutive decode steps near the 4096-slot cap (context 4000..4095):
    128 keys per attention split, four LDS tiles per block; with the f32
    cache and with the f16 one (the long-context stress is specified with an
    f16 N(0,1) cache; the oracle then rounds new K/V rows to f16 as well)."""
    print(f"[long] 1-layer engines, f16 KV {kv_f16}", flush=True)
    g = gpu_engine(n_layers=1, max_seq=4096, kv_f16=kv_f16)
    o = oracle_engine(n_layers=1, max_seq=4096)
    # an f16 K/V element whose f32 value sits near a rounding boundary can
    # round the other way (one f16 ulp, 2^-11 relative)
    a_tol, n_tol = (1e-2, 2e-3) if kv_f16 else (1e-3, 1e-3)
    try:
        if kv_f16:
            o.set_kv_f16(True)
        g.fill_kv_synthetic(SEED, 4000)
        fill_oracle_kv(o, SEED, 4000)
        g.position = 4000
        o.position = 4000
        for i, pos in enumerate((4000, 4001, 4002)):
            x = O.gen_f32(SEED + 40 + i, "input.hidden", 3072)
            _, gn = g.backbone_step(precomputed=x)
            o.backbone_step(precomputed=x)
            assert max_rel_err(g.debug_read("attn_out", 4096), o.buffer("attn_out")) < a_tol
            assert max_rel_err(gn, o.buffer("normed")) < n_tol, pos
        g.position = 4095
        o.position = 4095
        x = O.gen_f32(SEED + 50, "input.hidden", 3072)
        _, gn = g.backbone_step(precomputed=x)
        o.backbone_step(precomputed=x)
        assert max_rel_err(gn, o.buffer("normed")) < n_tol
        assert g.position == 4096
    finally:
        g.destroy()
        o.close()


def test_long_context_decode_26_layers_f32_kv():
    """The bench's long-context workload with the reference's f32 KV cache:
    the full 26-layer backbone decoding consecutive positions 3896..3899
    over a synthetic N(0,1) cache (122 keys per attention split, four LDS
    tiles per block).  Hidden states to the 1e-2 bar at every step."""
    print("[long] 26-layer engines, f32 KV, positions 3896..3899", flush=True)
    g = gpu_engine(n_layers=26, max_seq=4096)
    o = oracle_engine(n_layers=26, max_seq=4096)
    try:
        g.fill_kv_synthetic(SEED, 3896)
        fill_oracle_kv(o, SEED, 3896)
        g.position = 3896
        o.position = 3896
        for i in range(4):
            x = O.gen_f32(SEED + 70 + i, "input.hidden", 3072)
            _, gn = g.backbone_step(precomputed=x)
            o.backbone_step(precomputed=x)
            err = max_rel_err(gn, o.buffer("normed"))
            print(f"[long] position {3896 + i}: normed max rel err {err:.2e}", flush=True)
            assert err < 1e-2 and ref_allclose(gn, o.buffer("normed")), (i, err)
        assert g.position == o.position == 3900
    finally:
        g.destroy()
        o.close()


def test_long_context_decode_26_layers_f16_kv():
    """The long-context stress as specified: the full 26-layer backbone with
    the f16 KV cache, decoding consecutive positions 3896..3899 over a
    synthetic N(0,1) cache.  The cache is filled with the same f16 values on
    both sides (the oracle holds them exactly as f32), so only the rounding
    of each step's new K/V row to f16 can differ (one f16 ulp where the f32
    values of the two summation orders straddle a rounding boundary).
    Hidden states to the 1e-2 bar at every step."""
    print("[long] 26-layer engines, f16 KV, positions 3896..3899", flush=True)
    g = gpu_engine(n_layers=26, max_seq=4096, kv_f16=True)
    o = oracle_engine(n_layers=26, max_seq=4096)
    try:
        o.set_kv_f16(True)
        g.fill_kv_synthetic(SEED, 3896)
        fill_oracle_kv(o, SEED, 3896)
        g.position = 3896
        o.position = 3896
        for i in range(4):
            x = O.gen_f32(SEED + 60 + i, "input.hidden", 3072)
            _, gn = g.backbone_step(precomputed=x)
            o.backbone_step(precomputed=x)
            err = max_rel_err(gn, o.buffer("normed"))
            print(f"[long] position {3896 + i}: normed max rel err {err:.2e}", flush=True)
            assert err < 1e-2 and ref_allclose(gn, o.buffer("normed")), (i, err)
        assert g.position == o.position == 3900
    finally:
        g.destroy()
        o.close()
