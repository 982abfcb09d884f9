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

// classifyComponent (src/weights.ts:478-483)
function classifyComponent(name) {
  if (name.startsWith('acoustic_transformer.')) return 'fm';
  if (name.startsWith('audio_tokenizer.')) return 'codec';
  if (name.startsWith('layers.') || name.startsWith('norm.') || name.startsWith('mm_audio_embeddings.'))
    return 'backbone';
  return 'other';
}

// the tensor names of a safetensors file's header
function safetensorsNames(file) {
  const fd = fs.openSync(file, 'r');
  try {
    const len = Buffer.alloc(8);
    if (fs.readSync(fd, len, 0, 8, 0) !== 8) throw new Error(`${file}: not a safetensors file`);
    const n = Number(len.readBigUInt64LE(0));
    if (n === 0 || n > (64 << 20)) throw new Error(`${file}: not a safetensors file`);
    const hdr = Buffer.alloc(n);
    if (fs.readSync(fd, hdr, 0, n, 8) !== n) throw new Error(`${file}: short read of the header`);
    let obj;
    try { obj = JSON.parse(hdr.toString('utf8')); } catch (e) { throw new Error(`${file}: not a safetensors file`); }
    return Object.keys(obj).filter((k) => k !== '__metadata__');
  } finally {
    fs.closeSync(fd);
  }
}

class VoxtralEngine {
  /** new VoxtralEngine(EngineOptions), src/engine.ts:213-219, 301-304:
   *  config, maxSeqLen (4096), weightsUrl (here a local path: the default
   *  location of loadWeights / loadWeightsFromHF), onProgress(msg) (stage
   *  messages) and onWeightProgress(WeightLoadProgress) (the default
   *  per-tensor callback of loadWeights) */
  constructor(options) {
    options = options || {};
    this.config = options.config || null;
    this.maxSeqLen = options.maxSeqLen || 4096;
    this.weightsUrl = options.weightsUrl;
    this.onProgress = options.onProgress;
    this.onWeightProgress = options.onWeightProgress;
    this._h = null;
  }

  _say(msg) {
    if (this.onProgress) this.onProgress(msg);
  }

  /** init(), src/engine.ts:313: device + buffers (weights arrive next) */
  async init() {
    if (this._h) return;
    this._say('Creating the MI355X engine...');
    this._h = native.create(flattenConfig(this.config), this.maxSeqLen);
    this._say('Engine ready');
  }

  _handle() {
    if (!this._h) throw new Error('Engine not initialized. Call init() and loadWeights() first.');
    return this._h;
  }

  /** loadWeights(baseUrl, onProgress?), src/engine.ts:539-566, with a local
   *  path in place of the base URL (default: EngineOptions.weightsUrl):
   *   - a directory holding manifest.json: the reference's pre-extracted F16
   *     format (src/weights.ts:14-32, 317-369): per component (backbone, fm,
   *     codec) the tensors the manifest lists, f16 bits at offset/size of
   *     their .bin file, with the reference's WeightLoadProgress events
   *     ({loaded, total, component, tensor}: 0..3 of 'all' around the
   *     components, per component every 20 tensors and the last);
   *   - one .safetensors file, or a directory whose *.safetensors shards are
   *     loaded in name order: converted as the reference's loader converts
   *     (BF16 -> f16 by convertBF16toF16, F32 -> f16 by truncation, F16 as is),
   *     a WeightLoadProgress event after every tensor.
   *  onProgress defaults to EngineOptions.onWeightProgress.  Tensors the
   *  engine does not hold (codec tensors of an engine created without the
   *  decoder) are skipped.  Resolves to {loaded, skipped}. */
  async loadWeights(baseUrl, onProgress) {
    const location = baseUrl || this.weightsUrl;
    const cb = onProgress || this.onWeightProgress;
    if (typeof location !== 'string' || location.length === 0)
      throw new Error('loadWeights: pass a local directory (manifest.json or shards) or a .safetensors file');
    this._handle();
    this._say(`Loading weights from ${location}...`);
    let r;
    if (fs.statSync(location).isDirectory() && fs.existsSync(path.join(location, 'manifest.json'))) {
      r = this._loadManifest(location, cb);
    } else {
      r = this._loadSafetensors(location, cb ? (p) => cb({
        loaded: p.loaded, total: p.total, component: p.component, tensor: p.tensor,
      }) : null);
    }
    this._say(`Weights loaded: ${r.loaded} tensors (${r.skipped} skipped)`);
    return r;
  }

  /** loadWeightsFromHF(safetensorsUrl, onProgress?), src/engine.ts:569-586,
   *  with a local .safetensors file or directory of shards in place of the
   *  URL (default: EngineOptions.weightsUrl).  onProgress receives the
   *  reference's HFLoadProgress ({loaded, total, component, tensor, cached,
   *  bytesDownloaded}; src/weights.ts:465-472): first {component: 'init'},
   *  then one event per tensor in component order; cached is false and
   *  bytesDownloaded counts the bytes read from the files. */
  async loadWeightsFromHF(safetensorsUrl, onProgress) {
    const location = safetensorsUrl || this.weightsUrl;
    if (typeof location !== 'string' || location.length === 0)
      throw new Error('loadWeightsFromHF: pass a local .safetensors file or a directory of shards');
    this._handle();
    this._say(`Loading weights from ${location}...`);
    const r = this._loadSafetensors(location, onProgress ? (p) => onProgress(p) : null, true);
    this._say(`Weights loaded: ${r.loaded} tensors (${r.skipped} skipped)`);
    return r;
  }

  _shards(location) {
    let files = [location];
    if (fs.statSync(location).isDirectory())
      files = fs.readdirSync(location).filter((f) => f.endsWith('.safetensors')).sort()
        .map((f) => path.join(location, f));
    if (files.length === 0) throw new Error(`loadWeights: no .safetensors files in ${location}`);
    return files;
  }

  // every shard of location; progress(HFLoadProgress) after each tensor,
  // with loaded / total over all shards (total: the backbone, fm and codec
  // names of the headers, as loadWeightsFromHF counts them)
  _loadSafetensors(location, progress, initEvent) {
    const h = this._handle();
    const files = this._shards(location);
    let total = 0;
    if (progress) {
      for (const f of files) {
        for (const name of safetensorsNames(f)) {
          const c = classifyComponent(name);
          if (c !== 'other' && (c !== 'codec' || this._codec())) total++;
        }
      }
      if (initEvent)
        progress({ loaded: 0, total, component: 'init', tensor: 'Starting fresh download...',
          cached: false, bytesDownloaded: 0 });
    }
    const sum = { loaded: 0, skipped: 0 };
    let bytes = 0;
    for (const f of files) {
      const base = sum.loaded, bytes0 = bytes;
      const r = native.loadSafetensors(h, f, progress ? (loaded, t, component, tensor, b) => {
        bytes = bytes0 + b;
        progress({ loaded: base + loaded, total, component, tensor, cached: false, bytesDownloaded: bytes });
      } : null);
      sum.loaded += r.loaded;
      sum.skipped += r.skipped;
    }
    return sum;
  }

  // the pre-extracted F16 format: manifest.json + one .bin per component
  _loadManifest(dir, onProgress) {
    const h = this._handle();
    const log = onProgress || (() => {});
    let manifest;
    try {
      manifest = JSON.parse(fs.readFileSync(path.join(dir, 'manifest.json'), 'utf8'));
    } catch (e) {
      throw new Error(`Failed to load manifest: ${e.message}`);
    }
    if (!manifest || typeof manifest.tensors !== 'object')
      throw new Error('Failed to load manifest: no tensors');
    const steps = [['backbone', 'Loading backbone...'], ['fm', 'Loading FM transformer...'],
      ['codec', 'Loading codec decoder...']];
    const sum = { loaded: 0, skipped: 0 };
    const fds = new Map();
    try {
      steps.forEach(([component, msg], k) => {
        log({ loaded: k, total: 3, component: 'all', tensor: msg });
        const names = Object.keys(manifest.tensors).filter((n) => manifest.tensors[n].component === component);
        if (names.length === 0) return;
        const binFile = manifest.tensors[names[0]].file;
        log({ loaded: 0, total: names.length, component, tensor: `downloading ${binFile}...` });
        names.forEach((name, i) => {
          const info = manifest.tensors[name];
          if (info.dtype !== 'f16')
            throw new Error(`Unsupported dtype for ${name}: ${info.dtype} (the manifest format holds f16)`);
          if (!(info.size >= 0) || info.size % 2 !== 0 || !(info.offset >= 0))
            throw new Error(`${name}: bad offset ${info.offset} / size ${info.size}`);
          const file = path.join(dir, info.file);
          if (!fds.has(file)) fds.set(file, fs.openSync(file, 'r'));
          const buf = Buffer.alloc(info.size);
          if (fs.readSync(fds.get(file), buf, 0, info.size, info.offset) !== info.size)
            throw new Error(`Failed to download ${info.file}: short read of ${name}`);
          const f16 = new Uint16Array(buf.buffer, buf.byteOffset, info.size / 2);
          if (component === 'codec' && !this._codec()) {
            sum.skipped++;
          } else {
            native.loadTensor(h, name, f16, info.shape);
            sum.loaded++;
          }
          if (i % 20 === 0 || i === names.length - 1)
            log({ loaded: i + 1, total: names.length, component, tensor: name });
        });
      });
    } finally {
      for (const fd of fds.values()) fs.closeSync(fd);
    }
    const missing = native.missingTensor(h);
    if (missing !== null) throw new Error(`Missing weight: ${missing}`);
    log({ loaded: 3, total: 3, component: 'all', tensor: 'Done!' });
    return sum;
  }

  /** the same as loadWeights for a single safetensors file */
  loadSafetensors(file) {
    return native.loadSafetensors(this._handle(), file);
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
