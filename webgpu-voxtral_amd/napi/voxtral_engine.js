'use strict';
// VoxtralEngine over the MI355X HIP engine: the public surface of the
// reference's class (src/engine.ts:291-2632, types src/engine.ts:213-237)
// implemented on the Node-API addon voxtral_napi.node, which calls the C ABI
// of libvoxtral_amd.so (include/voxtral_engine.h).  Plain ES2019 so that it
// runs on the Node 12 of this image; voxtral_engine.d.ts carries the types.
const fs = require('fs');
const path = require('path');

const ADDON = process.env.VOXTRAL_NAPI || path.join(__dirname, '..', 'lib', 'voxtral_napi.node');
const native = require(ADDON);

const EMBED_TOKEN = 0;
const EMBED_AUDIO = 1;
const EMBED_PRECOMPUTED = 2;

// debugCodecDecode's intermediates in decoder order (VX_CODEC_STOP_* 0..9)
const CODEC_STOPS = ['concat', 'after_input_conv',
  'after_stage0_transformer', 'after_stage0_conv_up',
  'after_stage1_transformer', 'after_stage1_conv_up',
  'after_stage2_transformer', 'after_stage2_conv_up',
  'after_stage3_transformer', 'audio'];

// reference defaultConfig (src/types.ts:70-122), the fields the engine reads
function flattenConfig(config) {
  if (!config) return null;
  const b = config.backbone || {};
  const fm = config.fm || {};
  const out = {};
  const put = (k, v) => { if (v !== undefined) out[k] = v; };
  put('dim', b.dim);
  put('nLayers', b.n_layers);
  put('headDim', b.head_dim);
  put('hiddenDim', b.hidden_dim);
  put('nHeads', b.n_heads);
  put('nKvHeads', b.n_kv_heads);
  put('vocabSize', b.vocab_size);
  put('ropeTheta', b.rope_theta);
  put('normEps', b.norm_eps);
  put('fmLayers', fm.n_layers);
  put('nfe', fm.nfe);
  put('cfgAlpha', fm.cfg_alpha);
  put('kvF16', config.kvF16 ? 1 : undefined);
  put('codec', config.codec === false ? 0 : undefined);
  return out;
}

class VoxtralEngine {
  /** new VoxtralEngine({config?, maxSeqLen? = 4096}), src/engine.ts:301-304 */
  constructor(options) {
    options = options || {};
    this.config = options.config || null;
    this.maxSeqLen = options.maxSeqLen || 4096;
    this._h = null;
  }

  /** init(), src/engine.ts:313: device + buffers (weights arrive next) */
  async init() {
    if (this._h) return;
    this._h = native.create(flattenConfig(this.config), this.maxSeqLen);
  }

  _handle() {
    if (!this._h) throw new Error('Engine not initialized. Call init() and loadWeights() first.');
    return this._h;
  }

  /** loadWeights (src/engine.ts:539-566) with a local path in place of the
   *  base URL: one .safetensors file, or a directory whose *.safetensors
   *  shards are loaded in name order.  Tensors convert as the reference's
   *  loader converts them (BF16 -> f16 by convertBF16toF16, F32 -> f16 by
   *  truncation, F16 as is); codec-decoder tensors are skipped.
   *  Resolves to {loaded, skipped} summed over the shards. */
  async loadWeights(location) {
    if (typeof location !== 'string' || location.length === 0)
      throw new Error('loadWeights: pass a local .safetensors file or a directory of shards');
    const h = this._handle();
    let files = [location];
    if (fs.statSync(location).isDirectory())
      files = fs.readdirSync(location).filter((f) => f.endsWith('.safetensors')).sort()
        .map((f) => path.join(location, f));
    if (files.length === 0) throw new Error(`loadWeights: no .safetensors files in ${location}`);
    const total = { loaded: 0, skipped: 0 };
    for (const f of files) {
      const r = native.loadSafetensors(h, f);
      total.loaded += r.loaded;
      total.skipped += r.skipped;
    }
    return total;
  }

  /** the same, for a single file */
  loadSafetensors(file) {
    return native.loadSafetensors(this._handle(), file);
  }

  async loadWeightsFromHF(location) {
    return this.loadWeights(location);
  }

  /** one tensor of organizeWeights (src/engine.ts:659-743): f16 bits */
  loadTensor(name, f16, shape) {
    native.loadTensor(this._handle(), name, f16, shape);
  }

  /** every weight from the portable seeded generator (tests, benchmarks) */
  initSynthetic(seed, std) {
    native.initSynthetic(this._handle(), seed || 0, std === undefined ? 0.02 : std);
  }

  /** isReady, src/engine.ts:2054-2056 */
  get isReady() {
    return this._h !== null && native.isReady(this._h);
  }

  get position() {
    return native.position(this._handle());
  }

  set position(p) {
    native.position(this._handle(), p);
  }

  /** reset(), src/engine.ts:2323-2327 */
  reset() {
    native.reset(this._handle());
  }

  /** debugRead(name, count), src/engine.ts:2062-2067 */
  async debugRead(bufferName, count) {
    return native.read(this._handle(), bufferName, count === undefined ? 16 : count);
  }

  /** backboneStepAndRead, src/engine.ts:2333-2342: LM-head argmax */
  async backboneStepAndRead(tokenId, useAudioEmbedding) {
    const mode = useAudioEmbedding ? EMBED_AUDIO : EMBED_TOKEN;
    return native.backboneStep(this._handle(), tokenId, mode, null, true).argmax;
  }

  /** debugBackboneStepFull, src/engine.ts:2348-2357: W.normed */
  async debugBackboneStepFull(tokenId, useAudioEmbedding) {
    const mode = useAudioEmbedding ? EMBED_AUDIO : EMBED_TOKEN;
    return native.backboneStep(this._handle(), tokenId, mode, null, false).normed;
  }

  /** debugBackboneLayerByLayer(tokenId), src/engine.ts:2106-2287: one step
   *  with the embedding, each layer's attn_norm, attn_out (after the
   *  attention residual), ffn_norm and ffn_out (after the FFN residual),
   *  the final norm and the last hidden state */
  async debugBackboneLayerByLayer(tokenId) {
    const h = this._handle();
    const r = native.backboneLayers(h, tokenId, EMBED_TOKEN, null);
    const dim = r.embed.length, n = r.layers.length / (4 * dim);
    const at = (l, k) => r.layers.slice((4 * l + k) * dim, (4 * l + k + 1) * dim);
    const layers = [];
    for (let l = 0; l < n; l++) {
      layers.push({ attn_norm: at(l, 0), attn_out: at(l, 1), ffn_norm: at(l, 2), ffn_out: at(l, 3) });
    }
    return {
      embed: r.embed, layers, final_norm: native.read(h, 'normed', dim),
      hidden: layers[n - 1].ffn_out.slice(),
    };
  }

  /** backbone step on a precomputed embedding (src/engine.ts:847-854) */
  async backboneStepEmbedding(embedding) {
    return native.backboneStep(this._handle(), 0, EMBED_PRECOMPUTED, embedding, false).normed;
  }

  /** debugFMStep(debugNoise?), src/engine.ts:2363-2380 */
  async debugFMStep(debugNoise) {
    const r = native.fmForward(this._handle(), debugNoise || null);
    return { semantic_logits: r.semanticLogits, acoustic_codes: r.acousticCodes, x_final: r.xFinal };
  }

  /** fmStepAndRead, src/engine.ts:2386-2396 */
  async fmStepAndRead() {
    return native.fmForward(this._handle(), null).acousticCodes;
  }

  /**
   * generate(tokens, audioTokenStart, audioTokenCount, voiceEmbeddings,
   * maxFrames = 500, onFrame?, onStage?), src/engine.ts:2416-2616.  `audio`
   * is codecDecode of the generated frames (1920 samples each; empty for an
   * engine created with config.codec === false).  `options` (not in the
   * reference) selects sampling 'top_p' (default, the reference's),
   * 'top_p_host' or 'greedy', the seed that replaces Math.random, and
   * ignoreEos.
   */
  async generate(tokens, audioTokenStart, audioTokenCount, voiceEmbeddings, maxFrames,
    onFrame, onStage, options) {
    const opts = Object.assign({}, options || {}, { audio: this._codec() });
    return native.generate(this._handle(), tokens, audioTokenStart, audioTokenCount,
      voiceEmbeddings || null, maxFrames === undefined ? 500 : maxFrames, opts,
      onFrame || null, onStage || null);
  }

  /** codecDecode(semanticCodes, acousticCodes), src/engine.ts:1402-1713:
   *  codes [T] and [T * 36] -> 24 kHz samples [T * 1920] */
  async codecDecode(semanticCodes, acousticCodes) {
    return native.codecDecode(this._handle(), Uint32Array.from(semanticCodes),
      Uint32Array.from(acousticCodes));
  }

  /** debugCodecDecode, src/engine.ts:1719-1985: the decoder's intermediates
   *  by the reference's names */
  async debugCodecDecode(semanticCodes, acousticCodes) {
    const sem = Uint32Array.from(semanticCodes);
    const ac = Uint32Array.from(acousticCodes);
    const out = {};
    CODEC_STOPS.forEach((name, stop) => {
      out[name] = native.codecDecode(this._handle(), sem, ac, stop);
    });
    out.after_output_conv = out.audio;
    return out;
  }

  _codec() {
    return !(this.config && this.config.codec === false);
  }

  /** destroy(), src/engine.ts:2621-2632 */
  destroy() {
    if (this._h) native.destroy(this._h);
    this._h = null;
  }
}

module.exports = { VoxtralEngine, native, EMBED_TOKEN, EMBED_AUDIO, EMBED_PRECOMPUTED };
