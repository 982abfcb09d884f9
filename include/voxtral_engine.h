/*
 * voxtral_engine.h -- C ABI of the MI355X Voxtral frame-loop engine
 * (libvoxtral_amd.so).
 *
 * The library replaces the WebGPU engine of svenflow/webgpu-voxtral
 * (src/engine.ts, class VoxtralEngine) for the per-frame token loop: the
 * 26-layer backbone decode step and the flow-matching CFG Euler loop.  Every
 * entry point below names the reference method it stands in for.  Plain C
 * types only: host arrays are copied in and out; the engine owns all device
 * memory.
 *
 * Conventions
 *   - Every function returning int returns VX_OK (0) or a negative VX_E*
 *     code; vx_last_error() then holds the message (per handle; a NULL
 *     handle reads the message of the last failed vx_create).
 *   - A handle is not thread safe: one caller at a time.  All work of a
 *     handle runs in order on one HIP stream that the handle owns.
 *   - Weights are IEEE binary16 bit patterns, row-major [out, in], exactly
 *     the tensors the reference loads (src/engine.ts:659-743).
 */
#ifndef VOXTRAL_ENGINE_H
#define VOXTRAL_ENGINE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VX_OK 0
#define VX_E_INVALID -1    /* bad argument, shape or name */
#define VX_E_STATE -2      /* e.g. called before all weights are loaded */
#define VX_E_DEVICE -3     /* HIP runtime error */
#define VX_E_RANGE -4      /* position would pass max_seq_len */
#define VX_E_NOMEM -5

typedef struct vx_engine vx_engine;

/* Model constants, src/types.ts:70-122 (backbone + fm + the codec constant
 * the FSQ step reads).  The HIP kernels are specialised for the default
 * values; vx_create rejects other shapes. */
typedef struct vx_config {
  int32_t dim;             /* 3072 */
  int32_t n_layers;        /* 26 (1..26 accepted: single-layer workloads) */
  int32_t head_dim;        /* 128 */
  int32_t hidden_dim;      /* 9216 */
  int32_t n_heads;         /* 32 */
  int32_t n_kv_heads;      /* 8 */
  int32_t vocab_size;      /* 131072 */
  float rope_theta;        /* 1e6 */
  float norm_eps;          /* 1e-5 */
  int32_t fm_layers;       /* 3 */
  int32_t nfe;             /* 8 timesteps -> nfe-1 Euler updates */
  float cfg_alpha;         /* 1.2 */
  int32_t n_acoustic_out;  /* 36 */
  int32_t semantic_vocab;  /* 8320 */
  int32_t acoustic_levels; /* 21 */
  int32_t audio_vocab;     /* 9088 */
  /* KV cache element type (no reference field): 0 = f32, the reference's
   * KV precision (src/engine.ts:510-530), the default; 1 = f16, half the KV
   * traffic.  Rounding cached K/V rows to f16 perturbs hidden states by
   * more than 1e-2 after 26 random-weight layers, so parity with the
   * reference holds for 0 only. */
  int32_t kv_f16;
  /* Codec decoder (no reference field; the reference always has one,
   * src/engine.ts:1402-1713): 1 = its weights are part of the engine and
   * generate() returns audio, the default; 0 = the frame loop only. */
  int32_t codec;
} vx_config;

/* defaultConfig, src/types.ts:70-122 */
int vx_config_default(vx_config *cfg);

/* new VoxtralEngine({config, maxSeqLen}) + init(), src/engine.ts:301-340.
 * max_seq_len: KV slots per layer (reference default 4096). */
int vx_create(const vx_config *cfg, int32_t max_seq_len, vx_engine **out);

/* destroy(), src/engine.ts:2621-2632 */
void vx_destroy(vx_engine *e);

const char *vx_last_error(const vx_engine *e);

/* One tensor of loadWeights()/loadWeightsFromHF() + organizeWeights(),
 * src/engine.ts:539-586, 659-743.  `name` is the reference tensor name, e.g.
 * "layers.3.attention.wq.weight"; `shape` must match.  Unknown names are
 * VX_E_INVALID ("Missing weight" is reported by vx_is_ready()). */
int vx_load_tensor(vx_engine *e, const char *name, const uint16_t *f16,
                   size_t numel, const int64_t *shape, int32_t ndim);

/* No counterpart in the reference: fills every weight on the device from
 * the counter-based generator (seed, tensor name), mean 0 and std `std`
 * (norm gains: mean 1).  For synthetic benchmarks; bit-identical to the
 * CPU oracle's generator. */
int vx_init_synthetic(vx_engine *e, uint64_t seed, float std);

/* Copies a loaded weight back to the host (no reference counterpart; test
 * plumbing for generator and loader checks). */
int vx_read_tensor(vx_engine *e, const char *name, uint16_t *f16, size_t numel);

/* loadWeightsFromHF, src/engine.ts:569-586 with src/weights.ts:478-669,
 * from a local file instead of HTTP range requests: every tensor of the
 * safetensors file whose name the engine uses is converted to f16 with the
 * reference's rules (BF16: convertBF16toF16, src/weights.ts:94-138; F32:
 * float32ToFloat16, :222-232; F16 as is) and loaded.  Codec decoder tensors
 * (audio_tokenizer.*) and other names are skipped and counted.  Errors:
 * unreadable file or header, an unsupported dtype ("Unsupported dtype for
 * <name>: <dtype>"), a size or shape that differs from the engine's. */
int vx_load_safetensors(vx_engine *e, const char *path, int32_t *n_loaded,
                        int32_t *n_skipped);

/* Per-tensor progress of a weight load, the fields of HFLoadProgress /
 * WeightLoadProgress (src/weights.ts:149-154, 465-472): `loaded` of `total`
 * tensors the engine takes from the file, the tensor's component
 * (classifyComponent, src/weights.ts:478-483: backbone, fm, codec) and name,
 * and the bytes read from the file so far. */
typedef void (*vx_load_cb)(void *user, int32_t loaded, int32_t total,
                           const char *component, const char *tensor,
                           uint64_t bytes_read);
/* vx_load_safetensors with on_tensor (nullable) called after each tensor is
 * on the device, tensors in component order backbone, fm, codec as
 * loadWeightsFromHF orders them (src/weights.ts:520-523). */
int vx_load_safetensors_progress(vx_engine *e, const char *path,
                                 vx_load_cb on_tensor, void *user,
                                 int32_t *n_loaded, int32_t *n_skipped);
/* organizeWeights' "Missing weight: <name>" check (src/engine.ts:663-667):
 * 1 and the first weight not yet loaded (name truncated to cap bytes with a
 * terminating NUL), or 0 when every weight is loaded. */
int vx_missing_tensor(const vx_engine *e, char *name, int32_t cap);

/* The two conversions above, on the host (no device needed). */
void vx_bf16_to_f16(const uint16_t *bf16, uint16_t *f16, size_t n);
void vx_f32_to_f16_trunc(const float *f32, uint16_t *f16, size_t n);

/* isReady getter, src/engine.ts:2054-2056.  1 when every weight is loaded. */
int vx_is_ready(const vx_engine *e);

/* reset(), src/engine.ts:2323-2327: position = 0 (stale KV is never read). */
int vx_reset(vx_engine *e);
int32_t vx_position(const vx_engine *e);
int vx_set_position(vx_engine *e, int32_t pos);

/* Embedding source of a backbone step (src/engine.ts:814-854). */
#define VX_EMBED_TOKEN 0       /* row `token` of tok_embeddings */
#define VX_EMBED_AUDIO 1       /* row `token` of audio_codebook_embeddings */
#define VX_EMBED_PRECOMPUTED 2 /* `precomputed` f32[dim] replaces it */
#define VX_EMBED_CODES 3       /* multi-codebook sum of the device codes */

/* backboneStep + position++ (src/engine.ts:814-1042; public forms
 * backboneStepAndRead :2333-2342 and debugBackboneStepFull :2348-2357).
 * lm_head != 0 also runs the tied LM head and its argmax (written to
 * *argmax_out when not NULL).  normed_out (nullable) receives the final-norm
 * output f32[dim] (W.normed). */
int vx_backbone_step(vx_engine *e, int32_t token, int32_t embed_mode,
                     const float *precomputed, int32_t lm_head,
                     uint32_t *argmax_out, float *normed_out);

/* The prefill loop of generate(), src/engine.ts:2457-2472 (one
 * backboneStep per prompt token, voice rows replacing the embeddings of
 * tokens [audio_start, audio_start + audio_count)), run as batched MFMA
 * GEMMs over chunks of up to 256 tokens from the current position.  Leaves
 * the KV cache, the residual stream, W.normed (last token) and the position
 * as n_tokens single steps would (no LM head).  voice: f32[audio_count][dim]
 * or NULL. */
int vx_prefill(vx_engine *e, const int32_t *tokens, int32_t n_tokens,
               int32_t audio_start, int32_t audio_count, const float *voice);

/* debugBackboneLayerByLayer read points, src/engine.ts:2106-2287: one step
 * that also copies the hidden state after each attention residual and each
 * FFN residual into layer_out[n_layers][2][dim]. */
int vx_backbone_step_layers(vx_engine *e, int32_t token, int32_t embed_mode,
                            const float *precomputed, float *layer_out);

/* debugBackboneLayerByLayer, src/engine.ts:2106-2287, with all of its read
 * points: one step that copies the embedding (the first layer's input) into
 * embed[dim] and, per layer, the attention RMSNorm output, the hidden state
 * after the attention residual, the FFN RMSNorm output and the hidden state
 * after the FFN residual into layers[n_layers][4][dim] (either pointer may
 * be NULL, not both).  The final norm is W.normed afterwards (vx_read). */
int vx_debug_backbone_layers(vx_engine *e, int32_t token, int32_t embed_mode,
                             const float *precomputed, float *embed, float *layers);

/* fmForward (src/engine.ts:1240-1380; public form debugFMStep :2363-2380).
 * noise: f32[36] (debugNoise) or NULL for the engine's seeded generator.
 * Outputs (each nullable): semantic logits f32[8320], acoustic codes
 * u32[36], final x_t f32[36].  The unmasked tree argmax of the logits is
 * stored as the device semantic code (W.semantic_argmax). */
int vx_fm_forward(vx_engine *e, const float *noise, float *semantic_logits,
                  uint32_t *acoustic_codes, float *x_final);

/* writeBuffer(W.semantic_argmax), src/engine.ts:2574-2575, and the
 * teacher-forcing counterpart for the acoustic codes. */
int vx_set_semantic_code(vx_engine *e, uint32_t code);
int vx_set_acoustic_codes(vx_engine *e, const uint32_t *codes36);
int vx_get_codes(vx_engine *e, uint32_t *semantic, uint32_t *codes36);

/* debugRead(name, count), src/engine.ts:2062-2067.  Names: hidden, normed,
 * q, attn_out, gate (SwiGLU output), logits, semantic_logits, x_t,
 * velocity, v_uncond, fm_hidden (llm projection), fm_seq (6 x dim: cond
 * positions 0..2 then uncond), time_proj (table of nfe-1 rows). */
int vx_read(vx_engine *e, const char *buffer, float *dst, size_t count);

/* queue.writeBuffer into a work buffer (the reference's only host->device
 * activation path, e.g. src/engine.ts:1266-1274, 2574-2575); names:
 * "hidden" (next step input is not affected: steps embed first), "normed"
 * (input of the next vx_fm_forward -- teacher forcing). */
int vx_write(vx_engine *e, const char *buffer, const float *src, size_t count);

/* KV cache access (no reference counterpart; test and prefill plumbing).
 * Layout seen by the caller: [pos][n_kv_heads * head_dim] f32, the
 * reference's [maxSeq, 1024] row order (src/engine.ts:510-530).  With an
 * f16 cache, writes round to nearest even and reads widen exactly. */
int vx_write_kv(vx_engine *e, int32_t layer, int32_t which /*0=K,1=V*/,
                int32_t pos0, int32_t npos, const float *src);
int vx_read_kv(vx_engine *e, int32_t layer, int32_t which, int32_t pos0,
               int32_t npos, float *dst);
/* Fills positions [0, npos) of every layer's K and V with N(0,1) values
 * rounded to f16 from the generator (stream "kv.<layer>.k"/"kv.<layer>.v",
 * element index pos*1024 + c), held exactly in either cache type. */
int vx_fill_kv_synthetic(vx_engine *e, uint64_t seed, int32_t npos);

/* ----------------------------------------------------------- generate() */
/* Semantic-code sampling of generate() (src/engine.ts:2556-2567): the
 * logits masked (index 0, indices >= 8194), then sampleTopP(0.9, 0.8)
 * (src/engine.ts:247-289) with a seeded uniform instead of Math.random. */
#define VX_SAMPLE_TOP_P 0      /* top-p on the device: no logits readback */
#define VX_SAMPLE_GREEDY 1     /* masked argmax on the device */
#define VX_SAMPLE_TOP_P_HOST 2 /* the same top-p on the host (logits read back) */

typedef struct vx_generate_options {
  int32_t sampling;   /* VX_SAMPLE_* */
  double top_p;       /* 0.9 (a JS number in the reference) */
  double temperature; /* 0.8 */
  uint64_t seed;      /* noise + sampling seed (reference: Math.random) */
  int32_t ignore_eos; /* 1: run exactly max_frames (benchmarks) */
} vx_generate_options;

typedef struct vx_generate_stats {
  double backbone_ms; /* prefill (TTSResult.stats.backboneMs) */
  double fm_ms;       /* frame loop (stats.fmMs) */
  double codec_ms;    /* codec decode of the generated codes (0 without audio_out) */
  double total_ms;
  int32_t frames_generated;
} vx_generate_stats;

/* onFrame(frame, semanticCode, acousticCodes) and onStage(stage, doneMs)
 * of generate(), src/engine.ts:2416-2424.  stage: 0 backbone, 1 fm,
 * 2 codec; done_ms < 0 marks a stage start. */
typedef void (*vx_frame_cb)(void *user, int32_t frame, uint32_t semantic,
                            const uint32_t *acoustic36);
typedef void (*vx_stage_cb)(void *user, int32_t stage, double done_ms);

void vx_generate_options_default(vx_generate_options *o);

/* generate(tokens, audioTokenStart, audioTokenCount, voiceEmbeddings,
 * maxFrames, onFrame, onStage), src/engine.ts:2416-2616.  voice:
 * f32[audio_count][dim] or NULL.  semantic_out[max_frames] and
 * acoustic_out[max_frames][36] receive the codes; audio_out
 * f32[max_frames * VX_FRAME_SAMPLES] receives codecDecode of the generated
 * frames (TTSResult.audio; 1920 samples per frame).  All three are
 * nullable; audio_out needs an engine created with cfg.codec = 1.
 * After an EOS the engine holds what the EOS frame left, as after the
 * reference's loop: the position, the residual stream, normed, the semantic
 * logits, the codes, the FM noise frame counter and the top-p generator
 * state.  (The device-sampling modes run one frame ahead and undo it.)  The
 * FM scratch buffers (fm_hidden, x_history, velocities) are not restored:
 * they hold the discarded frame's values until the next FM pass. */
int vx_generate(vx_engine *e, const int32_t *tokens, int32_t n_tokens,
                int32_t audio_start, int32_t audio_count, const float *voice,
                int32_t max_frames, const vx_generate_options *opt,
                vx_frame_cb on_frame, vx_stage_cb on_stage, void *user,
                uint32_t *semantic_out, uint32_t *acoustic_out, float *audio_out,
                vx_generate_stats *stats);

/* ----------------------------------------------------------- tokenizer */
/* Byte-level BPE of TekkenTokenizer (src/tokenizer.ts:58-249), encoding
 * only.  Pre-tokenisation (the tekken.json regex pattern) stays with the
 * host's regex engine; the merge loop runs here.  Errors are reported
 * through vx_last_error(NULL). */
typedef struct vx_tokenizer vx_tokenizer;

/* constructor, src/tokenizer.ts:66-96: vocabulary entry i is the byte
 * string blob[offsets[i] .. offsets[i + 1]) (decoded token_bytes) with its
 * rank; token id = rank + num_special (default_num_special_tokens). */
int vx_tokenizer_create(const uint8_t *blob, const int64_t *offsets, const int32_t *ranks,
                        int32_t n, int32_t num_special, vx_tokenizer **out);
void vx_tokenizer_destroy(vx_tokenizer *t);

/* encode + bpeEncode over pre-tokenized pieces (src/tokenizer.ts:176-249): piece j
 * is the UTF-8 byte string bytes[offsets[j] .. offsets[j + 1]).  The ids of
 * all pieces, in order, go to out[0 .. *n_out); VX_E_RANGE (with *n_out
 * set) when cap is too small.  A part missing from the vocabulary encodes
 * as 0 (UNK), an empty piece as one UNK, as in the reference. */
int vx_tokenizer_encode_pieces(const vx_tokenizer *t, const uint8_t *bytes,
                               const int64_t *offsets, int32_t n_pieces, int32_t *out,
                               int64_t cap, int64_t *n_out);

/* ------------------------------------------------------- codec decoder */
#define VX_FRAME_SAMPLES 1920     /* 80 ms of 24 kHz audio per frame */
#define VX_CODEC_MAX_FRAMES 65536 /* 87 minutes of audio per call */
/* codecDecode(semanticCodes, acousticCodes), src/engine.ts:1402-1713:
 * semantic[n_frames], acoustic[n_frames][36] (values as generate() emits
 * them: semantic 2..8193 indexes the 8192-row VQ codebook directly, as the
 * reference's vqLookup does, rows past it read as zero; acoustic 2..22) ->
 * audio f32[n_frames * VX_FRAME_SAMPLES]. */
int vx_codec_decode(vx_engine *e, const uint32_t *semantic, const uint32_t *acoustic,
                    int32_t n_frames, float *audio);

/* debugCodecDecode (src/engine.ts:1719-1985): the decoder up to one of its
 * intermediates.  out must hold vx_codec_stop_count(n_frames, stop) floats. */
#define VX_CODEC_STOP_CONCAT 0      /* [T][292] VQ embedding | FSQ values */
#define VX_CODEC_STOP_INPUT_CONV 1  /* after_input_conv [T][1024] */
#define VX_CODEC_STOP_STAGE0 2      /* after_stage{s}_transformer: 2 + 2s; */
                                    /* after_stage{s}_conv_up: 3 + 2s (s < 3) */
#define VX_CODEC_STOP_AUDIO 9       /* audio [8T][240] */
int vx_codec_decode_debug(vx_engine *e, const uint32_t *semantic, const uint32_t *acoustic,
                          int32_t n_frames, int32_t stop, float *out, size_t out_count);
size_t vx_codec_stop_count(int32_t n_frames, int32_t stop);

/* sampleTopP on caller logits (test plumbing): logits f32[n] with indices
 * 0 and >= valid masked, n <= 9216.  *state: the splitmix64 state of the
 * uniform (advanced by one draw).  on_device != 0 runs the device kernel
 * used by generate(), else the host implementation. */
int vx_sample_top_p(vx_engine *e, const float *logits, int32_t n, int32_t valid,
                    double top_p, double temperature, uint64_t *state,
                    int32_t on_device, uint32_t *code);

/* No counterpart in the reference.  For callers that cannot allocate
 * device memory (tight serving loops, harnesses that forbid hipMalloc): the
 * device path of vx_sample_top_p, with no engine and no allocation.  Its
 * staging (logits, parameters, state, code: 37 KB) is a file-scope device
 * array of the library, one per GPU, so n is at most 9216 (larger n returns
 * VX_E_RANGE).  Runs on the null stream of the current device and waits for
 * it.  Calls from threads of one process take turns on a per-GPU lock;
 * calls from different processes that overlap on one GPU share the array
 * and race.  Errors are read with vx_last_error(NULL). */
int vx_sample_top_p_noalloc(const float *logits, int32_t n, int32_t valid,
                            double top_p, double temperature, uint64_t *state,
                            uint32_t *code);

/* ------------------------------------------------------ measurement */
/* No reference counterparts (the reference times on the CPU,
 * src/benchmark.ts:277-320).  Each runs on the handle's stream, bracketed
 * by HIP events, inputs resident in HBM. */

/* n backbone decode steps (graph replays); LM head off.  *ms = total event
 * time.  mode:
 *   VX_TIME_ADVANCE   each step starts from the residual stream the previous
 *                     step left; positions advance by n (the context grows);
 *   VX_TIME_HOLD      the same, but every step decodes at the current
 *                     position (reads the same number of keys, rewrites that
 *                     KV row) and the position stays;
 *   VX_TIME_FEEDBACK  positions advance, and each step's input embedding is
 *                     the previous step's W.normed, taken through the
 *                     precomputed-embedding path (src/engine.ts:847-854): a
 *                     prompt's decode tail fed with each frame's output. */
#define VX_TIME_ADVANCE 0
#define VX_TIME_HOLD 1
#define VX_TIME_FEEDBACK 2
int vx_time_backbone_steps(vx_engine *e, int32_t n, int32_t mode, float *ms);
/* n frames of the full loop (multi-codebook embed + backbone + FM, greedy
 * codes on the device, no EOS), as one graph replay each. */
int vx_time_frames(vx_engine *e, int32_t n, float *ms);

#define VX_KERNEL_QKV 0
#define VX_KERNEL_ATTN 1
#define VX_KERNEL_OPROJ 2
#define VX_KERNEL_GATEUP 3
#define VX_KERNEL_DOWN 4
/* flow-matching kernels: the four MFMA GEMMs, the attention, the Euler
 * step's input kernel */
#define VX_KERNEL_FM_QKV 5
#define VX_KERNEL_FM_ATTN 6
#define VX_KERNEL_FM_O 7
#define VX_KERNEL_FM_GATEUP 8
#define VX_KERNEL_FM_DOWN 9
#define VX_KERNEL_FM_STEP_IN 10
/* Average duration of one launch of a backbone or FM kernel (cycling over
 * the layers so no launch finds its weights in cache; FM kernels after one
 * full FM pass, on the buffers it leaves); *bytes = algorithmic HBM bytes of
 * one launch at the current position. */
int vx_time_kernel(vx_engine *e, int32_t kernel, int32_t iters, float *avg_us,
                   double *bytes);

/* Launch timeline of one decode step (no counterpart in the reference: a
 * measurement without a profiler).  Replays a copy of the held decode step's
 * graph reps times (the same kernels as VX_TIME_HOLD) in which every block
 * of every launch folds its start and end time on the GPU's 100 MHz wall
 * clock into its launch's slot.  stamps[2 i], stamps[2 i + 1] receive the
 * earliest block start and the latest block end of launch i of the last
 * replay: i = 6 l + k for layer l (k: 0 QKV, 1 attention partials,
 * 2 combine, 3 O, 4 gate/up, 5 down), then the final norm;
 * *n_out = 6 * n_layers + 1 launches, cap >= 2 * *n_out. */
int vx_debug_timeline(vx_engine *e, int32_t reps, uint64_t *stamps, int32_t cap,
                      int32_t *n_out);

int vx_synchronize(vx_engine *e);

#ifdef __cplusplus
}
#endif
#endif
