"""TekkenTokenizer (src/tokenizer.ts) over libvoxtral_amd's BPE encoder.

The class mirrors the reference's: built from a parsed tekken.json
(constructor, src/tokenizer.ts:66-96), with getVoiceNumTokens,
buildTTSPrompt, encode and voices.  Pre-tokenisation uses the pattern of
tekken.json (config.pattern) through the `regex` module, which reads the
\\p{...} classes of the JS 'u' flag; a pattern it cannot compile falls back
to \\S+|\\s+, as the reference's RegExp does.  Each piece is UTF-8 encoded
and merged by vx_tokenizer_encode_pieces (the byte-level BPE of bpeEncode,
src/tokenizer.ts:196-249).
"""
import base64
import ctypes
import json

import numpy as np
import regex

from . import VoxtralError, load_library

# special token ids, src/tokenizer.ts:14-26
TOKENS = {"UNK": 0, "BOS": 1, "EOS": 2, "INST": 3, "INST_END": 4, "AUDIO": 24,
          "BEGIN_AUDIO": 25, "OUTPUT_AUDIO": 26, "AUDIO_TO_TEXT": 35, "TEXT_TO_AUDIO": 36,
          "PAD": 11}

_FALLBACK = r"\S+|\s+"


def utf8(text):
    """UTF-8 bytes as TextEncoder gives them: a lone surrogate becomes U+FFFD."""
    try:
        return text.encode("utf-8")
    except UnicodeEncodeError:
        return text.encode("utf-16-le", "surrogatepass").decode("utf-16-le", "replace").encode("utf-8")


def _err(lib, rc):
    msg = lib.vx_last_error(None)
    return VoxtralError(rc, msg.decode() if msg else f"error {rc}")


class TekkenTokenizer:
    def __init__(self, data):
        lib = load_library()
        self._lib = lib
        self.num_special_tokens = int(data["config"]["default_num_special_tokens"])
        vocab = data["vocab"]
        pieces = [base64.b64decode(e["token_bytes"]) for e in vocab]
        offsets = np.zeros(len(pieces) + 1, np.int64)
        offsets[1:] = np.cumsum([len(p) for p in pieces])
        blob = np.frombuffer(b"".join(pieces) or b"\0", np.uint8)
        ranks = np.array([e["rank"] for e in vocab], np.int32)
        h = ctypes.c_void_p()
        rc = lib.vx_tokenizer_create(blob.ctypes.data, offsets.ctypes.data, ranks.ctypes.data,
                                     len(pieces), self.num_special_tokens, ctypes.byref(h))
        if rc:
            raise _err(lib, rc)
        self._h = h
        self.special_tokens = {st["token_str"]: st["rank"] for st in data.get("special_tokens", [])}
        try:
            self.pattern = regex.compile(data["config"]["pattern"])
        except (regex.error, KeyError, TypeError):
            self.pattern = regex.compile(_FALLBACK)
        audio = data.get("audio") or {}
        self.voice_num_tokens = dict(audio.get("voice_num_audio_tokens") or {})

    @classmethod
    def load(cls, path):
        """TekkenTokenizer.load (src/tokenizer.ts:101-105) from a local file."""
        with open(path, "rb") as f:
            return cls(json.loads(f.read()))

    def close(self):
        if getattr(self, "_h", None):
            self._lib.vx_tokenizer_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def voices(self):
        return list(self.voice_num_tokens)

    def get_voice_num_tokens(self, voice):
        """getVoiceNumTokens (src/tokenizer.ts:110-116)"""
        if voice not in self.voice_num_tokens:
            raise ValueError(f"Unknown voice: {voice}. Available: {', '.join(self.voice_num_tokens)}")
        return self.voice_num_tokens[voice]

    def encode(self, text):
        """encode (src/tokenizer.ts:176-188): regex pieces, then BPE."""
        pieces = [utf8(m.group(0)) for m in self.pattern.finditer(text)]
        if not pieces:
            return []
        offsets = np.zeros(len(pieces) + 1, np.int64)
        offsets[1:] = np.cumsum([len(p) for p in pieces])
        data = np.frombuffer(b"".join(pieces) or b"\0", np.uint8)
        cap = int(offsets[-1]) + len(pieces)  # at most one id per byte (one per empty piece)
        out = np.empty(max(cap, 1), np.int32)
        n = ctypes.c_int64()
        rc = self._lib.vx_tokenizer_encode_pieces(self._h, data.ctypes.data, offsets.ctypes.data,
                                                  len(pieces), out.ctypes.data, cap,
                                                  ctypes.byref(n))
        if rc:
            raise _err(self._lib, rc)
        return out[:n.value].tolist()

    def build_tts_prompt(self, text, voice):
        """buildTTSPrompt (src/tokenizer.ts:127-165):
        BOS [BEGIN_AUDIO] [AUDIO] x N [TEXT_TO_AUDIO] text [AUDIO_TO_TEXT] [BEGIN_AUDIO]"""
        n = self.get_voice_num_tokens(voice)
        tokens = [TOKENS["BOS"], TOKENS["BEGIN_AUDIO"]]
        start = len(tokens)
        tokens += [TOKENS["AUDIO"]] * n
        tokens.append(TOKENS["TEXT_TO_AUDIO"])
        tokens += self.encode(text)
        tokens += [TOKENS["AUDIO_TO_TEXT"], TOKENS["BEGIN_AUDIO"]]
        return {"tokens": tokens, "audioTokenStart": start, "audioTokenCount": n}
