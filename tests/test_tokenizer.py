"""Tekken tokenizer encoding (src/tokenizer.ts): the oracle's restatement of
bpeEncode pinned by hand-traced merges; the library's heap-based BPE
(vx_tokenizer_encode_pieces) against the oracle on fuzzed Unicode text over
a trained vocabulary; the TTS prompt layout; the Node class against the
Python one."""
import base64
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

import tekken_fixture as FX
import tekken_oracle as TO
from voxtral_amd.tokenizer import TOKENS, TekkenTokenizer, utf8

NS = 1000


def tiny(pattern=r"\S+|\s+"):
    """a=0 b=1 c=2 d=3 bc=4 ab=5 abc=6 aa=7; 'x' absent"""
    entries = [b"a", b"b", b"c", b"d", b"bc", b"ab", b"abc", b"aa"]
    return {"config": {"pattern": pattern, "default_num_special_tokens": NS},
            "vocab": [{"rank": i, "token_bytes": base64.b64encode(e).decode(), "token_str": ""}
                      for i, e in enumerate(entries)],
            "special_tokens": [], "audio": {"voice_num_audio_tokens": {"v": 3}}}


# hand-traced bpeEncode results (ids = rank + 1000, UNK = 0)
KNOWN = {
    "abcd": [6 + NS, 3 + NS],     # bc(4) < ab(5): [a,bc,d] -> abc(6): [abc,d]
    "aaaa": [7 + NS, 7 + NS],     # leftmost aa first: [aa,a,a] -> [aa,aa]; aaaa absent
    "aaa": [7 + NS, 0 + NS],
    "bcab": [4 + NS, 5 + NS],     # bc(4) then ab(5); "bcab" absent
    "x": [0],                     # single byte outside the vocabulary
    "ax": [0 + NS, 0],
    "cab": [2 + NS, 5 + NS],
}


@pytest.mark.parametrize("text", list(KNOWN))
def test_oracle_known_answers(text):
    o = TO.TekkenOracle(tiny())
    assert o.encode(text, utf8) == KNOWN[text]


def test_oracle_empty_piece_is_unk():
    # an empty piece has no parts: the reference returns [UNK]
    assert TO.bpe_encode(b"", {b"a": 0}, NS) == [0]


@pytest.mark.parametrize("text", list(KNOWN))
def test_library_known_answers(text):
    assert TekkenTokenizer(tiny()).encode(text) == KNOWN[text]


def test_library_encode_pieces_edge_cases():
    t = TekkenTokenizer(tiny())
    assert t.encode("") == []
    # whitespace pieces hold bytes outside the tiny vocabulary: UNK each
    assert t.encode("abcd abcd\n") == KNOWN["abcd"] + [0] + KNOWN["abcd"] + [0]
    # an empty piece through the C ABI: one UNK
    import ctypes
    lib = t._lib
    off = np.array([0, 0, 4], np.int64)
    data = np.frombuffer(b"abcd", np.uint8)
    out = np.empty(8, np.int32)
    n = ctypes.c_int64()
    assert lib.vx_tokenizer_encode_pieces(t._h, data.ctypes.data, off.ctypes.data, 2,
                                          out.ctypes.data, 8, ctypes.byref(n)) == 0
    assert out[:n.value].tolist() == [0] + KNOWN["abcd"]
    # too small an output: VX_E_RANGE with the needed count
    assert lib.vx_tokenizer_encode_pieces(t._h, data.ctypes.data, off.ctypes.data, 2,
                                          out.ctypes.data, 2, ctypes.byref(n)) != 0
    assert n.value == 3


def fuzz_texts(seed, n):
    rng = np.random.default_rng(seed)
    pool = list("abcdefghijklmnopqrstuvwxyz ABCDEFGHIJ  0123456789.,;:!?'\"-/\\()~\n\t") + \
        list("éèüößñ¿¡ЖжЯ東京タワー語🎵🎶👍́ 　")
    words = FX.CORPUS.split()
    out = []
    for _ in range(n):
        if rng.random() < 0.5:
            s = "".join(rng.choice(pool) for _ in range(rng.integers(0, 60)))
        else:
            s = " ".join(rng.choice(words) for _ in range(rng.integers(1, 20)))
        out.append(s)
    return out


@pytest.fixture(scope="module")
def trained():
    return FX.build()


def test_library_matches_oracle_on_fuzzed_text(trained):
    t = TekkenTokenizer(trained)
    o = TO.TekkenOracle(trained)
    assert len(trained["vocab"]) > 350  # 254 bytes + every corpus word merged
    merged_any = False
    for s in fuzz_texts(0, 300) + [FX.CORPUS, FX.CORPUS[:500] * 4, "~" * 9, "a\ud800b"]:
        got, ref = t.encode(s), o.encode(s, utf8)
        assert got == ref, s
        merged_any |= any(i >= NS + 256 for i in got)
    assert merged_any


def test_fallback_pattern_and_prompt(trained):
    bad = dict(trained, config=dict(trained["config"], pattern="(?<unclosed"))
    t, o = TekkenTokenizer(bad), TO.TekkenOracle(bad)
    s = "Grüße  aus\nMünchen ~~"
    assert [m.group(0) for m in t.pattern.finditer(s)] == ["Grüße", "  ", "aus", "\n", "München", " ", "~~"]
    assert t.encode(s) == o.encode(s, utf8)
    p = TekkenTokenizer(trained).build_tts_prompt("Hello there.", "ar_male")
    assert p == TO.TekkenOracle(trained).build_tts_prompt("Hello there.", "ar_male", utf8)
    toks = p["tokens"]
    assert (p["audioTokenStart"], p["audioTokenCount"]) == (2, 67)
    assert toks[:2] == [TOKENS["BOS"], TOKENS["BEGIN_AUDIO"]]
    assert toks[2:69] == [TOKENS["AUDIO"]] * 67 and toks[69] == TOKENS["TEXT_TO_AUDIO"]
    assert toks[-2:] == [TOKENS["AUDIO_TO_TEXT"], TOKENS["BEGIN_AUDIO"]]
    with pytest.raises(ValueError, match="Unknown voice: x. Available: neutral_female, ar_male"):
        TekkenTokenizer(trained).build_tts_prompt("hi", "x")


ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
JS = os.path.join(ROOT, "webgpu-voxtral_amd", "napi", "voxtral_tokenizer.js")
ADDON = os.path.join(ROOT, "webgpu-voxtral_amd", "lib", "voxtral_napi.node")


@pytest.mark.skipif(shutil.which("node") is None or not os.path.exists(ADDON),
                    reason="node or the built addon is not available")
def test_node_class_matches_python(trained, tmp_path):
    path = tmp_path / "tekken.json"
    path.write_text(json.dumps(trained))
    texts = fuzz_texts(1, 80) + [FX.CORPUS]
    script = f"""
const {{ TekkenTokenizer }} = require({json.dumps(JS)});
TekkenTokenizer.load({json.dumps(str(path))}).then((t) => {{
  const texts = {json.dumps(texts)};
  const enc = texts.map((s) => t.encode(s));
  const p = t.buildTTSPrompt('Hello there.', 'neutral_female');
  let err = '';
  try {{ t.getVoiceNumTokens('nobody'); }} catch (e) {{ err = e.message; }}
  console.log(JSON.stringify({{ enc, p, err, voices: t.voices }}));
}});
"""
    r = subprocess.run(["node", "-e", script], capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout.strip().splitlines()[-1])
    t = TekkenTokenizer(trained)
    assert out["enc"] == [t.encode(s) for s in texts]
    assert out["p"] == t.build_tts_prompt("Hello there.", "neutral_female")
    assert out["err"] == "Unknown voice: nobody. Available: neutral_female, ar_male"
    assert out["voices"] == t.voices
