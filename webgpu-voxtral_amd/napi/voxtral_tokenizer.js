'use strict';
// TekkenTokenizer (src/tokenizer.ts:58-257) on the Node-API addon: the same
// class surface (constructor(data), load, getVoiceNumTokens, buildTTSPrompt,
// encode, voices).  Pre-tokenisation runs the tekken.json pattern through
// JS RegExp with the reference's 'gu' flags and /\S+|\s+/gu fallback; the
// byte-level BPE merge runs in libvoxtral_amd (vx_tokenizer_encode_pieces).
const fs = require('fs');
const { native } = require('./voxtral_engine.js');

// special token ids, src/tokenizer.ts:14-26
const TOKENS = Object.freeze({
  UNK: 0, BOS: 1, EOS: 2, INST: 3, INST_END: 4, AUDIO: 24, BEGIN_AUDIO: 25,
  OUTPUT_AUDIO: 26, AUDIO_TO_TEXT: 35, TEXT_TO_AUDIO: 36, PAD: 11,
});

// n byte strings -> one Uint8Array + Int32Array offsets[n + 1]
function packBytes(buffers) {
  const offsets = new Int32Array(buffers.length + 1);
  let total = 0;
  buffers.forEach((b, i) => { total += b.length; offsets[i + 1] = total; });
  const blob = new Uint8Array(Math.max(total, 1));
  buffers.forEach((b, i) => blob.set(b, offsets[i]));
  return { blob, offsets };
}

class TekkenTokenizer {
  /** constructor(data: parsed tekken.json), src/tokenizer.ts:66-96 */
  constructor(data) {
    this.numSpecialTokens = data.config.default_num_special_tokens;
    const vocab = data.vocab || [];
    const { blob, offsets } = packBytes(vocab.map((e) => Buffer.from(e.token_bytes, 'base64')));
    const ranks = Int32Array.from(vocab.map((e) => e.rank));
    this._h = native.tokenizerCreate(blob, offsets, ranks.length ? ranks : new Int32Array(1),
      this.numSpecialTokens);
    this.specialTokens = new Map((data.special_tokens || []).map((s) => [s.token_str, s.rank]));
    try {
      this.pattern = new RegExp(data.config.pattern, 'gu');
    } catch (e) {
      this.pattern = /\S+|\s+/gu;
    }
    const counts = (data.audio && data.audio.voice_num_audio_tokens) || {};
    this.voiceNumTokens = new Map(Object.entries(counts));
  }

  /** load(url) of the reference, src/tokenizer.ts:101-105, from a local file */
  static async load(path) {
    return new TekkenTokenizer(JSON.parse(fs.readFileSync(path, 'utf8')));
  }

  /** getVoiceNumTokens, src/tokenizer.ts:110-116 */
  getVoiceNumTokens(voice) {
    const n = this.voiceNumTokens.get(voice);
    if (n === undefined)
      throw new Error(`Unknown voice: ${voice}. Available: ${[...this.voiceNumTokens.keys()].join(', ')}`);
    return n;
  }

  /** buildTTSPrompt, src/tokenizer.ts:127-165 */
  buildTTSPrompt(text, voice) {
    const n = this.getVoiceNumTokens(voice);
    const tokens = [TOKENS.BOS, TOKENS.BEGIN_AUDIO];
    const audioTokenStart = tokens.length;
    for (let i = 0; i < n; i++) tokens.push(TOKENS.AUDIO);
    tokens.push(TOKENS.TEXT_TO_AUDIO);
    for (const t of this.encode(text)) tokens.push(t);
    tokens.push(TOKENS.AUDIO_TO_TEXT, TOKENS.BEGIN_AUDIO);
    return { tokens, audioTokenStart, audioTokenCount: n };
  }

  /** encode, src/tokenizer.ts:176-188: regex pieces, UTF-8, BPE */
  encode(text) {
    this.pattern.lastIndex = 0;
    const pieces = [];
    for (const m of text.matchAll ? text.matchAll(this.pattern) : matchAllCompat(text, this.pattern))
      pieces.push(Buffer.from(m[0], 'utf8'));
    if (pieces.length === 0) return [];
    const { blob, offsets } = packBytes(pieces);
    return Array.from(native.tokenizerEncode(this._h, blob, offsets));
  }

  /** voices, src/tokenizer.ts:254-256 */
  get voices() {
    return [...this.voiceNumTokens.keys()];
  }
}

// String.prototype.matchAll arrived in Node 12; a global-regex exec loop for
// older runtimes (empty matches advance by one code point, as matchAll does)
function* matchAllCompat(text, re) {
  const r = new RegExp(re.source, re.flags);
  let m;
  while ((m = r.exec(text)) !== null) {
    yield m;
    if (m[0].length === 0) r.lastIndex += text.codePointAt(r.lastIndex) > 0xffff ? 2 : 1;
  }
}

module.exports = { TekkenTokenizer, TOKENS };
