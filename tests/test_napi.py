"""The Node-API binding (webgpu-voxtral_amd/napi): the reference's
VoxtralEngine surface in Node over the C ABI.  CPU: the addon loads and
exports the API, and library errors arrive as JS Errors.  GPU: generate()
through Node equals generate() through the Python binding, with every
onFrame call delivered before the promise settles (src/engine.ts:2584)."""
import json
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
JS = os.path.join(ROOT, "webgpu-voxtral_amd", "napi", "voxtral_engine.js")
ADDON = os.path.join(ROOT, "webgpu-voxtral_amd", "lib", "voxtral_napi.node")

pytestmark = pytest.mark.skipif(shutil.which("node") is None or not os.path.exists(ADDON),
                                reason="node or the built addon is not available")


def run_node(script, timeout=120):
    p = subprocess.run(["node", "-e", script], capture_output=True, text=True, timeout=timeout,
                       cwd=ROOT)
    assert p.returncode == 0, p.stderr
    return p.stdout


def test_addon_exports_and_errors():
    out = run_node(f"""
const m = require({json.dumps(JS)});
const names = Object.keys(m.native).sort();
const e = new m.VoxtralEngine({{config: {{backbone: {{n_layers: 1}}}}, maxSeqLen: 64}});
let ready = e.isReady;
let msg = '';
try {{ e.reset(); }} catch (err) {{ msg = err.message; }}
e.init().then(() => console.log(JSON.stringify({{names, ready, msg, init: 'ok'}})),
              (err) => console.log(JSON.stringify({{names, ready, msg, init: err.message}})));
""")
    r = json.loads(out.strip().splitlines()[-1])
    assert r["names"] == sorted(["create", "destroy", "loadTensor", "loadSafetensors", "codecDecode",
                                 "tokenizerCreate", "tokenizerEncode",
                                 "initSynthetic", "isReady", "missingTensor",
                                 "reset", "position", "backboneStep", "backboneLayers", "fmForward",
                                 "setSemanticCode", "read", "generate"])
    assert r["ready"] is False
    assert r["msg"].startswith("Engine not initialized")
    # without a GPU the library's own error; with one, init succeeds
    assert r["init"] in ("ok", "No HIP device")


@pytest.mark.gpu
def test_generate_through_node_matches_python():
    tokens = [1, 25, 24, 24, 35, 500, 24]
    voice = 7
    script = f"""
const m = require({json.dumps(JS)});
(async () => {{
  const e = new m.VoxtralEngine({{config: {{backbone: {{n_layers: 2}}}}, maxSeqLen: 64}});
  await e.init();
  e.initSynthetic(0, 0.02);
  const voice = new Float32Array(2 * 3072);
  for (let i = 0; i < voice.length; i++) voice[i] = ((i * {voice}) % 13 - 6) * 0.0625;
  const frames = [];
  const stages = [];
  let settled = false, late = 0;
  const r = await e.generate({json.dumps(tokens)}, 2, 2, voice, 5,
    (f, s, codes) => {{ if (settled) late++; frames.push([f, s, Array.from(codes)]); }},
    (st, ms) => stages.push([st, ms === undefined ? null : 1]),
    {{sampling: 'greedy', seed: 3, ignoreEos: true}});
  settled = true;
  const dec = await e.codecDecode(r.semanticCodes, [].concat(...r.acousticCodes));
  const redecoded = dec.length === r.audio.length && dec.every((v, i) => v === r.audio[i]);
  const normed = await e.debugBackboneStepFull(24);
  const lbl = await e.debugBackboneLayerByLayer(24);
  const pick = (a) => Array.from(a.slice(0, 8));
  const layerHeads = lbl.layers.map((L) => [pick(L.attn_norm), pick(L.attn_out), pick(L.ffn_norm),
                                            pick(L.ffn_out)]);
  const hiddenIsLast = lbl.hidden.every((v, i) => v === lbl.layers[1].ffn_out[i]);
  e.destroy();
  console.log(JSON.stringify({{sem: r.semanticCodes, ac: r.acousticCodes, n: r.stats.framesGenerated,
                               redecoded,
                               frames, stages, late, audio: r.audio.length,
                               audio_head: Array.from(r.audio.slice(0, 64)), normed0: normed[0],
                               lbl_embed: pick(lbl.embed), lbl_layers: layerHeads,
                               lbl_final: pick(lbl.final_norm), lbl_hidden_last: hiddenIsLast}}));
}})().catch((err) => {{ console.error(err); process.exit(3); }});
"""
    print("[napi] node generate, 2 layers, 5 frames", flush=True)
    r = json.loads(run_node(script, timeout=300).strip().splitlines()[-1])

    import numpy as np
    import voxtral_amd as V
    g = V.VoxtralEngine(V.default_config(n_layers=2), max_seq_len=64).init()
    try:
        g.init_synthetic(0, 0.02)
        vo = (((np.arange(2 * 3072) * voice) % 13 - 6) * 0.0625).astype(np.float32)  # exact in both
        py = g.generate(tokens, 2, 2, vo, 5, sampling="greedy", seed=3, ignore_eos=True)
        normed = g.debug_backbone_step_full(24)
        lbl = g.debug_backbone_layer_by_layer(24)
    finally:
        g.destroy()
    assert r["n"] == 5 and r["sem"] == py["semanticCodes"] and r["ac"] == py["acousticCodes"]
    assert [f[0] for f in r["frames"]] == list(range(5)) and r["late"] == 0
    assert [f[1] for f in r["frames"]] == r["sem"] and [f[2] for f in r["frames"]] == r["ac"]
    assert r["stages"][0] == ["backbone", None] and r["stages"][-1][0] == "codec"
    # TTSResult.audio: codecDecode of the 5 frames, as through Python
    assert r["audio"] == 5 * 1920 == py["audio"].size
    assert r["redecoded"]
    # Every kernel of the codec is the library's own (no vendor GEMM whose
    # pick depends on which shared library a process loads), and each GEMM's
    # K-slice partials are added in a fixed order: the node process and this
    # one decode bit-identical audio.
    head = np.float32(r["audio_head"])
    assert np.array_equal(head, py["audio"][:64])
    # debugBackboneStepFull and debugBackboneLayerByLayer through Node: the
    # same kernels on the same state as through Python, bit for bit
    assert np.float32(r["normed0"]) == normed[0]
    assert np.array_equal(np.float32(r["lbl_embed"]), lbl["embed"][:8])
    names = ("attn_norm", "attn_out", "ffn_norm", "ffn_out")
    assert len(r["lbl_layers"]) == 2
    for l, got in enumerate(r["lbl_layers"]):
        for k, name in enumerate(names):
            assert np.array_equal(np.float32(got[k]), lbl["layers"][l][name][:8]), (l, name)
    assert np.array_equal(np.float32(r["lbl_final"]), lbl["final_norm"][:8])
    assert r["lbl_hidden_last"]


@pytest.mark.gpu
def test_load_weights_from_a_directory_of_shards(tmp_path):
    """loadWeights(dir): every *.safetensors shard in name order, counts
    summed; the engine then holds the converted weights."""
    import numpy as np
    from test_gpu_loader import to_bf16_bits, write_safetensors
    import voxtral_amd as V
    rng = np.random.default_rng(11)
    fn = (1 + rng.standard_normal(3072) * 0.1).astype(np.float32)
    write_safetensors(tmp_path / "model-00001-of-00002.safetensors",
                      {"layers.0.ffn_norm.weight": ("BF16", to_bf16_bits(fn)),
                       "audio_tokenizer.x": ("F32", np.zeros(2, np.float32))})
    write_safetensors(tmp_path / "model-00002-of-00002.safetensors",
                      {"norm.weight": ("F32", fn)})
    (tmp_path / "README").write_text("not a shard")
    script = f"""
const m = require({json.dumps(JS)});
(async () => {{
  const e = new m.VoxtralEngine({{config: {{backbone: {{n_layers: 1}}}}, maxSeqLen: 16}});
  await e.init();
  e.initSynthetic(0, 0.02);
  const r = await e.loadWeights({json.dumps(str(tmp_path))});
  let err = '';
  try {{ await e.loadWeights({json.dumps(str(tmp_path / "README"))}); }} catch (x) {{ err = x.message; }}
  const normed = await e.debugBackboneStepFull(24);
  e.destroy();
  console.log(JSON.stringify({{r, err, normed: Array.from(normed.slice(0, 8))}}));
}})().catch((err) => {{ console.error(err); process.exit(3); }});
"""
    print("[napi] loadWeights over two shards", flush=True)
    r = json.loads(run_node(script, timeout=300).strip().splitlines()[-1])
    assert r["r"] == {"loaded": 2, "skipped": 1}
    assert "not a safetensors file" in r["err"]
    g = V.VoxtralEngine(V.default_config(n_layers=1), max_seq_len=16).init()
    try:
        g.init_synthetic(0, 0.02)
        g.load_tensor("layers.0.ffn_norm.weight", V.bf16_to_f16(to_bf16_bits(fn)), [3072])
        g.load_tensor("norm.weight", V.f32_to_f16_trunc(fn), [3072])
        _, normed = g.backbone_step(24)
    finally:
        g.destroy()
    assert np.array_equal(np.float32(r["normed"]), normed[:8])


def write_manifest_dir(d, components):
    """The reference's pre-extracted F16 format (src/weights.ts:14-32): one
    .bin per component, manifest.json listing each tensor's file, offset,
    size, shape, dtype and component.  components: {component: {name: f16}}"""
    import numpy as np
    tensors = {}
    for comp, ts in components.items():
        blob, off = bytearray(), 0
        for name, arr in ts.items():
            b = np.ascontiguousarray(arr, np.float16).tobytes()
            tensors[name] = {"file": f"{comp}.bin", "offset": off, "size": len(b),
                             "padded_size": len(b), "shape": list(np.shape(arr)), "dtype": "f16",
                             "component": comp}
            blob += b
            off += len(b)
        (d / f"{comp}.bin").write_bytes(bytes(blob))
    (d / "manifest.json").write_text(json.dumps({"format": "f16", "source": "test",
                                                 "total_tensors": len(tensors), "tensors": tensors}))


@pytest.mark.gpu
def test_load_weights_manifest_and_progress(tmp_path):
    """loadWeights(baseUrl, onProgress) of the reference's manifest format
    (src/engine.ts:539-566, src/weights.ts:317-369) with its
    WeightLoadProgress events, EngineOptions.onWeightProgress / onProgress /
    weightsUrl (src/engine.ts:213-219), loadWeightsFromHF's HFLoadProgress
    events (src/weights.ts:465-472, 520-523, 629-636), and organizeWeights'
    "Missing weight" error (src/engine.ts:663-667)."""
    import numpy as np
    from test_gpu_loader import to_bf16_bits, write_safetensors
    import voxtral_amd as V
    rng = np.random.default_rng(12)
    fn = (1 + rng.standard_normal(3072) * 0.1).astype(np.float16)
    an = (1 + rng.standard_normal(3072) * 0.1).astype(np.float16)
    mdir = tmp_path / "m"
    mdir.mkdir()
    write_manifest_dir(mdir, {
        "backbone": {"layers.0.ffn_norm.weight": fn, "norm.weight": an},
        "fm": {"acoustic_transformer.norm.weight": an},
        "codec": {"audio_tokenizer.decoder.x": np.zeros(4, np.float16)}})
    st = tmp_path / "w.safetensors"
    sn = (1 + rng.standard_normal(3072) * 0.1).astype(np.float32)
    write_safetensors(st, {"layers.0.attention_norm.weight": ("BF16", to_bf16_bits(sn)),
                           "acoustic_transformer.layers.0.ffn_norm.weight": ("F32", sn),
                           "audio_tokenizer.y": ("F32", np.zeros(2, np.float32)),
                           "norm.weight": ("F16", an)})
    script = f"""
const m = require({json.dumps(JS)});
(async () => {{
  const msgs = [], wev = [], hev = [];
  const e = new m.VoxtralEngine({{config: {{backbone: {{n_layers: 1}}, codec: false}}, maxSeqLen: 16,
    weightsUrl: {json.dumps(str(mdir))}, onProgress: (s) => msgs.push(s), onWeightProgress: (p) => wev.push(p)}});
  await e.init();
  e.initSynthetic(0, 0.02);
  const r = await e.loadWeights();
  const r2 = await e.loadWeightsFromHF({json.dumps(str(st))}, (p) => hev.push(p));
  const normed = await e.debugBackboneStepFull(24);
  e.destroy();
  const f = new m.VoxtralEngine({{config: {{backbone: {{n_layers: 1}}, codec: false}}, maxSeqLen: 16}});
  await f.init();
  let missing = '';
  try {{ await f.loadWeights({json.dumps(str(mdir))}); }} catch (x) {{ missing = x.message; }}
  f.destroy();
  console.log(JSON.stringify({{r, r2, msgs, wev, hev, missing, normed: Array.from(normed.slice(0, 8))}}));
}})().catch((err) => {{ console.error(err); process.exit(3); }});
"""
    print("[napi] loadWeights: manifest + progress", flush=True)
    r = json.loads(run_node(script, timeout=300).strip().splitlines()[-1])
    assert r["r"] == {"loaded": 3, "skipped": 1}
    assert r["r2"] == {"loaded": 3, "skipped": 1}
    w = r["wev"]
    assert w[0] == {"loaded": 0, "total": 3, "component": "all", "tensor": "Loading backbone..."}
    assert w[1] == {"loaded": 0, "total": 2, "component": "backbone", "tensor": "downloading backbone.bin..."}
    assert w[2] == {"loaded": 1, "total": 2, "component": "backbone", "tensor": "layers.0.ffn_norm.weight"}
    assert w[3] == {"loaded": 2, "total": 2, "component": "backbone", "tensor": "norm.weight"}
    assert w[4]["tensor"] == "Loading FM transformer..." and w[-1] == {
        "loaded": 3, "total": 3, "component": "all", "tensor": "Done!"}
    h = r["hev"]
    assert h[0]["component"] == "init" and h[0]["loaded"] == 0 and h[0]["total"] == 3
    # one event per tensor, component order backbone, fm (codec skipped: no decoder)
    assert [(x["loaded"], x["component"], x["tensor"]) for x in h[1:]] == [
        (1, "backbone", "layers.0.attention_norm.weight"), (2, "backbone", "norm.weight"),
        (3, "fm", "acoustic_transformer.layers.0.ffn_norm.weight")]
    assert all(x["total"] == 3 and x["cached"] is False for x in h)
    b = [x["bytesDownloaded"] for x in h]
    assert b == sorted(b) and b[-1] <= st.stat().st_size
    assert any("Loading weights from" in s for s in r["msgs"])
    assert r["missing"].startswith("Missing weight: ")
    g = V.VoxtralEngine(V.default_config(n_layers=1, codec=0), max_seq_len=16).init()
    try:
        g.init_synthetic(0, 0.02)
        g.load_tensor("layers.0.ffn_norm.weight", fn.view(np.uint16), [3072])
        g.load_tensor("norm.weight", an.view(np.uint16), [3072])
        g.load_tensor("acoustic_transformer.norm.weight", an.view(np.uint16), [3072])
        g.load_tensor("layers.0.attention_norm.weight", V.bf16_to_f16(to_bf16_bits(sn)), [3072])
        g.load_tensor("acoustic_transformer.layers.0.ffn_norm.weight", V.f32_to_f16_trunc(sn), [3072])
        _, normed = g.backbone_step(24)
        events = []
        g.init_synthetic(1, 0.02)
        assert g.load_safetensors(st, events.append) == (3, 1)
        assert [e["tensor"] for e in events] == ["layers.0.attention_norm.weight", "norm.weight",
                                                 "acoustic_transformer.layers.0.ffn_norm.weight"]
        assert g.missing_tensor() is None
    finally:
        g.destroy()
    assert np.array_equal(np.float32(r["normed"]), normed[:8])


def test_numeric_arguments_are_range_checked():
    """Numbers that cannot be what the C ABI takes (NaN, fractions, values
    outside int32, negative frame counts or seeds) throw RangeError before
    any cast; no GPU is needed for these checks, which come first."""
    out = run_node(f"""
const m = require({json.dumps(JS)});
const n = m.native;
const res = {{}};
const tryit = (k, f) => {{ try {{ f(); res[k] = 'ok'; }} catch (e) {{ res[k] = e.constructor.name + ': ' + e.message; }} }};
tryit('create_nan', () => n.create({{nLayers: NaN}}, 64));
tryit('create_frac', () => n.create({{nLayers: 1.5}}, 64));
tryit('create_big', () => n.create(null, 2 ** 40));
console.log(JSON.stringify(res));
""")
    r = json.loads(out.strip().splitlines()[-1])
    assert r["create_nan"] == "RangeError: nLayers out of range"
    assert r["create_frac"] == "RangeError: nLayers out of range"
    assert r["create_big"] == "RangeError: maxSeqLen out of range"


@pytest.mark.gpu
def test_calls_during_a_pending_generate():
    """While generate() runs on the worker thread, a second generate()
    rejects, other calls throw, and destroy() is deferred until the pending
    generate() has completed: it still resolves, and the handle is dead
    afterwards.  Out-of-range options reject before anything runs."""
    script = f"""
const m = require({json.dumps(JS)});
(async () => {{
  const e = new m.VoxtralEngine({{config: {{backbone: {{n_layers: 2}}}}, maxSeqLen: 64}});
  await e.init();
  e.initSynthetic(0, 0.02);
  const out = {{}};
  const msg = async (f) => {{ try {{ await f(); return 'ok'; }} catch (x) {{ return x.constructor.name + ': ' + x.message; }} }};
  out.bad_frames = await msg(() => e.generate([1, 25, 24], 2, 0, null, -1));
  out.bad_seed = await msg(() => e.generate([1, 25, 24], 2, 0, null, 2, null, null, {{seed: 0.5}}));
  out.bad_temp = await msg(() => e.generate([1, 25, 24], 2, 0, null, 2, null, null, {{temperature: 0}}));
  out.bad_topp = await msg(() => e.generate([1, 25, 24], 2, 0, null, 2, null, null, {{topP: NaN}}));
  const p = e.generate([1, 25, 24, 24, 35, 500, 24], 2, 0, null, 6, null, null,
                       {{sampling: 'greedy', seed: 1, ignoreEos: true}});
  out.second = await msg(() => e.generate([1, 25, 24], 2, 0, null, 2));
  out.reset = await msg(() => e.reset());
  out.step = await msg(() => e.debugBackboneStepFull(24));
  out.ready = e.isReady;
  const h = e._h;
  e.destroy();
  out.destroyed_early = await msg(() => m.native.reset(h));
  const r = await p;
  out.frames = r.stats.framesGenerated;
  out.after = await msg(() => m.native.reset(h));
  console.log(JSON.stringify(out));
}})().catch((err) => {{ console.error(err); process.exit(3); }});
"""
    print("[napi] calls during a pending generate", flush=True)
    r = json.loads(run_node(script, timeout=300).strip().splitlines()[-1])
    assert r["bad_frames"] == "RangeError: maxFrames out of range"
    assert r["bad_seed"] == "RangeError: seed out of range"
    assert r["bad_temp"].startswith("Error: ") and "temperature" in r["bad_temp"]
    assert r["bad_topp"].startswith("Error: ") and "top_p" in r["bad_topp"]
    assert r["second"] == "Error: generate() is still running on this engine"
    assert r["reset"] == "Error: generate() is still running on this engine"
    assert r["step"] == "Error: generate() is still running on this engine"
    assert r["ready"] is True
    assert r["frames"] == 6
    assert r["destroyed_early"] == r["after"] == "Error: engine destroyed"
