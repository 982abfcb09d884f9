"""Pure-Python restatement of the reference's Tekken tokenizer encoding
(src/tokenizer.ts): encode :176-188 and bpeEncode :196-249, with the
buildTTSPrompt layout :127-165.

TEST INFRASTRUCTURE ONLY: the parity checker for the library's BPE encoder
(vx_tokenizer_encode_pieces).  Only tests/ import it.

bpeEncode, as the reference writes it: the piece's UTF-8 bytes start as
one part each; every pass scans all adjacent pairs for the concatenation
with the lowest vocabulary rank (strict <, so the leftmost wins ties),
merges that one pair, and scans again until no adjacent pair is in the
vocabulary.  Ids are rank + num_special_tokens; a part outside the
vocabulary, and an empty piece, is UNK (0).  Quadratic per piece: small
inputs only.
"""
import base64

import regex

UNK, BOS, AUDIO, BEGIN_AUDIO, AUDIO_TO_TEXT, TEXT_TO_AUDIO = 0, 1, 24, 25, 35, 36


def bpe_encode(piece_bytes, bytes_to_rank, num_special):
    parts = [bytes([b]) for b in piece_bytes]
    if len(parts) <= 1:
        r = bytes_to_rank.get(parts[0]) if parts else None
        return [r + num_special if r is not None else UNK]
    while len(parts) > 1:
        best_rank, best = None, -1
        for i in range(len(parts) - 1):
            r = bytes_to_rank.get(parts[i] + parts[i + 1])
            if r is not None and (best_rank is None or r < best_rank):
                best_rank, best = r, i
        if best < 0:
            break
        parts = parts[:best] + [parts[best] + parts[best + 1]] + parts[best + 2:]
    return [bytes_to_rank[p] + num_special if p in bytes_to_rank else UNK for p in parts]


class TekkenOracle:
    def __init__(self, data):
        self.num_special = data["config"]["default_num_special_tokens"]
        self.bytes_to_rank = {base64.b64decode(e["token_bytes"]): e["rank"] for e in data["vocab"]}
        try:
            self.pattern = regex.compile(data["config"]["pattern"])
        except (regex.error, KeyError, TypeError):
            self.pattern = regex.compile(r"\S+|\s+")
        self.voices = dict((data.get("audio") or {}).get("voice_num_audio_tokens") or {})

    def pieces(self, text):
        return [m.group(0) for m in self.pattern.finditer(text)]

    def encode(self, text, to_bytes):
        out = []
        for p in self.pieces(text):
            out += bpe_encode(to_bytes(p), self.bytes_to_rank, self.num_special)
        return out

    def build_tts_prompt(self, text, voice, to_bytes):
        n = self.voices[voice]
        toks = [BOS, BEGIN_AUDIO] + [AUDIO] * n + [TEXT_TO_AUDIO] + self.encode(text, to_bytes)
        return {"tokens": toks + [AUDIO_TO_TEXT, BEGIN_AUDIO], "audioTokenStart": 2,
                "audioTokenCount": n}
