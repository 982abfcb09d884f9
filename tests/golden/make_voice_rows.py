"""Writes tests/golden/ar_male_voice_rows64.f32: the first 64 rows of the
reference's real voice embedding models/voxtral-tts/voice_embedding_f32/
ar_male.bin (raw little-endian f32, [rows][3072]; 67 rows in the file).
These rows are what generate() splices over the [AUDIO] prompt positions
(src/engine.ts:2436-2465, src/tokenizer.ts:136-145).  The file is data: it is
copied as bytes, nothing of the reference is run.

Run from the repository root: python tests/golden/make_voice_rows.py
"""
import hashlib
import os
import sys

import numpy as np

SRC = "/root/reference/models/voxtral-tts/voice_embedding_f32/ar_male.bin"
ROWS, DIM = 64, 3072
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ar_male_voice_rows64.f32")


def main():
    a = np.fromfile(SRC, dtype="<f4")
    if a.size % DIM:
        sys.exit(f"{SRC}: {a.size} floats is not a multiple of {DIM}")
    rows = a.reshape(-1, DIM)[:ROWS]
    rows.astype("<f4").tofile(OUT)
    print(f"{OUT}: {rows.shape[0]} of {a.size // DIM} rows, sha256 "
          f"{hashlib.sha256(rows.astype('<f4').tobytes()).hexdigest()}")


if __name__ == "__main__":
    main()
