// Types of voxtral_engine.js: the reference's VoxtralEngine surface
// (src/engine.ts:213-237, 291-2632) for the per-frame token loop.

export interface VoxtralConfig {
  backbone?: {
    dim?: number; n_layers?: number; head_dim?: number; hidden_dim?: number;
    n_heads?: number; n_kv_heads?: number; vocab_size?: number;
    rope_theta?: number; norm_eps?: number;
  };
  fm?: { n_layers?: number; nfe?: number; cfg_alpha?: number };
  /** KV cache element type: false f32 (the reference's), true f16 */
  kvF16?: boolean;
  /** false: no codec decoder (generate() returns empty audio) */
  codec?: boolean;
}

/** src/weights.ts:149-154 */
export interface WeightLoadProgress {
  loaded: number;
  total: number;
  component: string;
  tensor: string;
}

/** src/weights.ts:465-472 */
export interface HFLoadProgress {
  loaded: number;
  total: number;
  component: string;
  tensor: string;
  /** always false here: the weights come from local files */
  cached: boolean;
  /** bytes read from the files so far */
  bytesDownloaded: number;
}

/** src/engine.ts:213-219 */
export interface EngineOptions {
  config?: VoxtralConfig;
  maxSeqLen?: number;
  /** default location of loadWeights / loadWeightsFromHF (a local path) */
  weightsUrl?: string;
  /** stage messages (engine creation, weight loading) */
  onProgress?: (msg: string) => void;
  /** default per-tensor callback of loadWeights */
  onWeightProgress?: (progress: WeightLoadProgress) => void;
}

export interface TTSResult {
  semanticCodes: number[];
  acousticCodes: number[][];
  /** codecDecode of the generated frames: 1920 samples of 24 kHz audio each */
  audio: Float32Array;
  stats: {
    backboneMs: number;
    fmMs: number;
    codecMs: number;
    totalMs: number;
    framesGenerated: number;
  };
}

export interface GenerateOptions {
  /** 'top_p' (the reference's sampling, on the device), 'top_p_host' (the same on the host), 'greedy' */
  sampling?: 'top_p' | 'top_p_host' | 'greedy';
  topP?: number;
  temperature?: number;
  seed?: number;
  ignoreEos?: boolean;
}

export declare class VoxtralEngine {
  constructor(options?: EngineOptions);
  init(): Promise<void>;
  /** a local directory in place of the base URL: manifest.json + .bin files (the
   *  pre-extracted f16 format), or *.safetensors shards; or one .safetensors file */
  loadWeights(baseUrl?: string, onProgress?: (progress: WeightLoadProgress) => void):
    Promise<{ loaded: number; skipped: number }>;
  /** a local .safetensors file (or directory of shards) in place of the URL */
  loadWeightsFromHF(safetensorsUrl?: string, onProgress?: (progress: HFLoadProgress) => void):
    Promise<{ loaded: number; skipped: number }>;
  loadSafetensors(file: string): { loaded: number; skipped: number };
  loadTensor(name: string, f16: Uint16Array, shape: number[]): void;
  initSynthetic(seed?: number, std?: number): void;
  readonly isReady: boolean;
  position: number;
  reset(): void;
  debugRead(bufferName: string, count?: number): Promise<Float32Array>;
  backboneStepAndRead(tokenId: number, useAudioEmbedding?: boolean): Promise<number>;
  debugBackboneStepFull(tokenId: number, useAudioEmbedding?: boolean): Promise<Float32Array>;
  debugBackboneLayerByLayer(tokenId: number): Promise<{
    embed: Float32Array;
    layers: Array<{
      attn_norm: Float32Array;
      attn_out: Float32Array;
      ffn_norm: Float32Array;
      ffn_out: Float32Array;
    }>;
    final_norm: Float32Array;
    hidden: Float32Array;
  }>;
  backboneStepEmbedding(embedding: Float32Array): Promise<Float32Array>;
  debugFMStep(debugNoise?: Float32Array): Promise<{
    semantic_logits: Float32Array;
    acoustic_codes: Uint32Array;
    x_final: Float32Array;
  }>;
  fmStepAndRead(): Promise<Uint32Array>;
  codecDecode(semanticCodes: ArrayLike<number>, acousticCodes: ArrayLike<number>): Promise<Float32Array>;
  debugCodecDecode(semanticCodes: ArrayLike<number>, acousticCodes: ArrayLike<number>): Promise<Record<string, Float32Array>>;
  generate(
    tokens: number[],
    audioTokenStart: number,
    audioTokenCount: number,
    voiceEmbeddings: Float32Array | null,
    maxFrames?: number,
    onFrame?: (frame: number, semanticCode: number, acousticCodes: Uint32Array) => void,
    onStage?: (stage: 'backbone' | 'fm' | 'codec', doneMs?: number) => void,
    options?: GenerateOptions,
  ): Promise<TTSResult>;
  destroy(): void;
}
