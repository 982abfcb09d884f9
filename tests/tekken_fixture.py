"""A synthetic tekken.json for tokenizer tests (the real file is not
shipped with the reference): byte tokens at ranks 0-255 (a few bytes left
out, so UNK appears), then BPE merges learned greedily from a corpus
(most frequent adjacent pair, ties to the smaller byte string), and the
pre-tokenisation pattern of Mistral's Tekken v7 tokenizer.  Built
deterministically; no reference code is involved."""
import base64
import collections

import regex

# Tekken pre-tokenisation pattern (word-like runs with an optional leading
# non-letter, single digits, punctuation runs, newline runs, whitespace)
PATTERN = (r"[^\r\n\p{L}\p{N}]?[\p{Lu}\p{Lt}\p{Lm}\p{Lo}\p{M}]*[\p{Ll}\p{Lm}\p{Lo}\p{M}]+|"
           r"[^\r\n\p{L}\p{N}]?[\p{Lu}\p{Lt}\p{Lm}\p{Lo}\p{M}]+[\p{Ll}\p{Lm}\p{Lo}\p{M}]*|"
           r"\p{N}| ?[^\s\p{L}\p{N}]+[\r\n/]*|\s*[\r\n]+|\s+(?!\S)|\s+")

CORPUS = ("The quick brown fox jumps over the lazy dog. Voxtral speaks: bonjour, "
          "¿qué tal? Grüße aus München! 東京タワーへ行きます。 It's 2026, and 12.5 frames "
          "per second make 24 kHz audio.\n\nNew paragraph -- with dashes/slashes, "
          "émojis 🎵🎶 and tabs\tinside. ") * 3

LEFT_OUT = (0x7E, 0xC0)  # '~' and a byte that never starts valid UTF-8


def build(n_merges=300, num_special=1000, voices=None, pattern=PATTERN):
    ranks = {bytes([b]): b for b in range(256) if b not in LEFT_OUT}
    words = [list(bytes([c]) for c in m.group(0).encode("utf-8"))
             for m in regex.finditer(PATTERN, CORPUS)]
    nxt = 256
    for _ in range(n_merges):
        counts = collections.Counter()
        for w in words:
            for a, b in zip(w, w[1:]):
                counts[a + b] += 1
        if not counts:
            break
        best = min(counts, key=lambda k: (-counts[k], k))
        if counts[best] < 2:
            break
        ranks[best] = nxt
        nxt += 1
        for w in words:
            i = 0
            while i < len(w) - 1:
                if w[i] + w[i + 1] == best:
                    w[i:i + 2] = [best]
                i += 1
    vocab = [{"rank": r, "token_bytes": base64.b64encode(b).decode(),
              "token_str": b.decode("utf-8", "replace")} for b, r in sorted(ranks.items(), key=lambda x: x[1])]
    return {
        "config": {"pattern": pattern, "num_vocab_tokens": len(vocab),
                   "default_vocab_size": len(vocab) + num_special,
                   "default_num_special_tokens": num_special, "version": "v7"},
        "vocab": vocab,
        "special_tokens": [{"rank": 0, "token_str": "<unk>", "is_control": True},
                           {"rank": 1, "token_str": "<s>", "is_control": True},
                           {"rank": 24, "token_str": "[AUDIO]", "is_control": True}],
        "audio": {"sampling_rate": 24000, "frame_rate": 12.5,
                  "voice_num_audio_tokens": voices or {"neutral_female": 218, "ar_male": 67}},
    }
