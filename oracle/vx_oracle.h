/*
 * vx_oracle.h -- CPU restatement of the reference Voxtral frame loop.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * engine and the CPU baseline that bench.py reports beside it.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product (webgpu-voxtral_amd) never links or calls it.
 *
 * Every kernel restates one WGSL shader of the reference with the same f32
 * arithmetic and the same per-workgroup reduction order (256 strided lane
 * partials followed by a shared-memory tree); the orchestration restates the
 * TypeScript engine.  Citations are to files of svenflow/webgpu-voxtral.
 *
 * Parity status of each function (how it is pinned) is listed in the header
 * of vx_oracle.c.
 */
#ifndef VX_ORACLE_H
#define VX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* src/types.ts:70-122 (defaultConfig), backbone + fm parts. */
typedef struct vxo_config {
  int dim;            /* 3072 */
  int n_layers;       /* 26 */
  int head_dim;       /* 128 */
  int hidden_dim;     /* 9216 */
  int n_heads;        /* 32 */
  int n_kv_heads;     /* 8 */
  int vocab_size;     /* 131072 */
  float rope_theta;   /* 1e6 */
  float norm_eps;     /* 1e-5 */
  int fm_layers;      /* 3 */
  int nfe;            /* 8 timesteps -> 7 Euler updates */
  float cfg_alpha;    /* 1.2 */
  int n_acoustic_out; /* 36 */
  int semantic_vocab; /* 8320 */
  int acoustic_levels;/* 21 (codec.acoustic_codebook_size) */
  int audio_vocab;    /* 9088 rows of audio_codebook_embeddings */
} vxo_config;

void vxo_default_config(vxo_config *c);

/* ---------------------------------------------------------------- numbers */
uint16_t vxo_f32_to_f16(float f);   /* IEEE binary16, round-to-nearest-even */
float vxo_f16_to_f32(uint16_t h);
uint64_t vxo_splitmix64_next(uint64_t *state);
uint64_t vxo_name_stream(const char *name); /* FNV-1a 64 of a tensor name */
/* Counter-based normal variate: Irwin-Hall sum of 12 uniforms (20 bits each)
 * taken from outputs 4*idx..4*idx+3 of the splitmix64 stream keyed by
 * (seed, stream); exact in f32, identical on any IEEE machine. */
float vxo_normal(uint64_t seed, uint64_t stream, uint64_t idx);
/* Box-Muller Gaussian (the FM noise), bit-identical to the device's */
float vxo_gauss(uint64_t seed, uint64_t stream, uint64_t idx);
void vxo_gen_gauss_f32(uint64_t seed, uint64_t stream, size_t n, float *out);
void vxo_gen_f32(uint64_t seed, uint64_t stream, size_t n, float mean,
                 float std, float *out);
void vxo_gen_f16(uint64_t seed, uint64_t stream, size_t n, float mean,
                 float std, uint16_t *out);

/* ---------------------------------------------------------------- kernels */
void vxo_matvec_f16(const uint16_t *A, const float *x, float *y, int M, int K);
void vxo_rmsnorm(const float *x, const uint16_t *w, float *y, int dim, float eps);
void vxo_embedding(const uint16_t *table, int token, int dim, float *out);
void vxo_rope(float *qk, int head_dim, int pos, int n_heads, float theta);
void vxo_attn_scores(const float *q, const float *kcache, float *scores,
                     int n_heads, int n_kv_heads, int head_dim, int seq_len);
void vxo_softmax(float *scores, int n_heads, int seq_len);
void vxo_attn_value(const float *scores, const float *vcache, float *out,
                    int n_heads, int n_kv_heads, int head_dim, int seq_len);
void vxo_swiglu(float *gate, const float *up, int n);
void vxo_time_embedding(float *out, int dim, float t);
void vxo_cfg_combine(float *v_cond, const float *v_uncond, int n, float alpha);
void vxo_euler_step(float *x, const float *v, int n, float dt);
void vxo_fsq_quantize(const float *x, uint32_t *codes, int n, int levels,
                      int offset);
uint32_t vxo_argmax(const float *x, int n);
void vxo_multi_codebook_embed(const uint16_t *table, uint32_t semantic_code,
                              const uint32_t *acoustic_codes, int dim,
                              float *out);
void vxo_bi_attention(const float *q, const float *k, const float *v,
                      float *scores, float *out, int n_heads, int n_kv_heads,
                      int head_dim, int seq_len);

/* ---------------------------------------------------------------- engine */
typedef struct vxo_engine vxo_engine;

vxo_engine *vxo_create(const vxo_config *cfg, int max_seq);
void vxo_destroy(vxo_engine *e);
/* Binds a weight by its reference tensor name (src/engine.ts:659-743).  The
 * caller keeps `data` alive.  Returns 0, or -1 for an unknown name. */
int vxo_set_weight(vxo_engine *e, const char *name, const uint16_t *data);
/* Allocates and fills every weight from the synthetic generator. */
int vxo_init_synthetic(vxo_engine *e, uint64_t seed, float std);
/* Fills/returns a named tensor element count (0 if unknown). */
size_t vxo_weight_numel(const vxo_engine *e, const char *name);
const uint16_t *vxo_weight(const vxo_engine *e, const char *name);
int vxo_is_ready(const vxo_engine *e);

void vxo_reset(vxo_engine *e);
/* on != 0: new K/V rows are stored rounded to f16 (the reference keeps
 * f32; the HIP engine keeps f16 as the benchmark configurations specify). */
void vxo_set_kv_f16(vxo_engine *e, int on);
int vxo_position(const vxo_engine *e);
void vxo_set_position(vxo_engine *e, int pos);
float *vxo_buffer(vxo_engine *e, const char *name, int *count);
float *vxo_kv(vxo_engine *e, int layer, int which /*0=k,1=v*/);
uint32_t *vxo_acoustic_codes(vxo_engine *e);
uint32_t vxo_semantic_argmax(const vxo_engine *e);
void vxo_set_semantic_code(vxo_engine *e, uint32_t code);
void vxo_set_acoustic_codes(vxo_engine *e, const uint32_t *codes);
uint32_t vxo_argmax_result(const vxo_engine *e);

/* One backbone step at the current position (src/engine.ts:814-1042),
 * then position++.  mode: 0 = token embedding, 1 = audio-table embedding,
 * 2 = `precomputed` row replaces the embedding.  lm_head != 0 also runs the
 * tied LM head + argmax (dead work in generate()). */
void vxo_backbone_step(vxo_engine *e, int token, int mode,
                       const float *precomputed, int lm_head);
/* Same step; when layer_out is not NULL it receives, per layer, the hidden
 * state after the attention residual and after the FFN residual
 * ([n_layers][2][dim], the debugBackboneLayerByLayer read points,
 * src/engine.ts:2106-2287). */
void vxo_backbone_step_ex(vxo_engine *e, int token, int mode,
                          const float *precomputed, int lm_head,
                          float *layer_out);
/* Same step with the read points of debugBackboneLayerByLayer
 * (src/engine.ts:2106-2287): embed [dim] (the embedding lookup, or the
 * precomputed row) and layers [n_layers][4][dim] = attn_norm, attn_out
 * (after the attention residual), ffn_norm, ffn_out (after the FFN
 * residual); either may be NULL.  No LM head. */
void vxo_backbone_step_debug(vxo_engine *e, int token, int mode,
                             const float *precomputed, float *embed,
                             float *layers);
/* multiCodebookEmbed of the engine's semantic + acoustic codes into hidden
 * (src/engine.ts:2499-2531), then a backbone step on it. */
void vxo_backbone_step_codes(vxo_engine *e);
/* src/engine.ts:1240-1380 with debugNoise = noise (required). */
void vxo_fm_forward(vxo_engine *e, const float *noise);
/* Optimal dataflow: CFG branches and the 3 positions batched per weight
 * read, time projection hoisted out of the frame.  Same arithmetic per
 * output element as vxo_fm_forward. */
void vxo_fm_forward_batched(vxo_engine *e, const float *noise);
/* generate() up to the codec decode (src/engine.ts:2416-2585) with the greedy
 * masked semantic code, device-stream noise and optional teacher forcing;
 * returns framesGenerated (see vx_oracle.c for the outputs). */
int vxo_generate(vxo_engine *e, const int32_t *tokens, int n_tokens, int audio_start,
                 int audio_count, const float *voice, int max_frames, uint64_t noise_seed,
                 int ignore_eos, const uint32_t *forced_sem, const uint32_t *forced_ac,
                 int n_forced, uint32_t *sem_out, uint32_t *ac_out, float *x_out,
                 float *normed_out, float *logits_out);

/* ------------------------------------------------------- codec decoder */
/* vx_oracle_codec.c: codecDecode (src/engine.ts:1402-1713) and its shaders
 * (src/shaders.ts:817-1110, 1432-1868). */
void vxo_normalize_codebook(const uint16_t *sum, const uint16_t *usage, uint16_t *out,
                            int n_entries, int dim, float eps);
void vxo_vq_lookup(const uint32_t *codes, const uint16_t *cb, float *out, int T, int dim,
                   int n_entries);
void vxo_fsq_dequant(const uint32_t *codes, float *out, int n, int levels, int offset);
void vxo_causal_conv1d(const float *in, const uint16_t *w, const uint16_t *g, float *out,
                       int c_in, int c_out, int kernel, int n_frames, int stride);
void vxo_conv_transpose_scale(const uint16_t *w, const uint16_t *g, float *scale, int c_in,
                              int c_out, int kernel);
void vxo_conv_transpose1d(const float *in, const uint16_t *w, const float *scale, float *out,
                          int c_in, int c_out, int kernel, int n_out, int stride);
void vxo_batched_rmsnorm(const float *in, const uint16_t *w, float *out, int dim, int T,
                         float eps);
void vxo_batched_matvec_f16(const uint16_t *A, const float *in, float *out, int M, int K,
                            int T);
void vxo_qk_norm(float *data, const uint16_t *w, int n_heads, int head_dim, int T, float eps);
void vxo_codec_attention(const float *q, const float *k, const float *v, float *out,
                         int n_heads, int head_dim, int T, int W);

typedef struct vxo_codec vxo_codec;
vxo_codec *vxo_codec_create(void);
void vxo_codec_destroy(vxo_codec *c);
int vxo_codec_n_weights(const vxo_codec *c);
const char *vxo_codec_weight_name(const vxo_codec *c, int i);
size_t vxo_codec_weight_numel(const vxo_codec *c, const char *name);
const uint16_t *vxo_codec_weight(const vxo_codec *c, const char *name);
int vxo_codec_set_weight(vxo_codec *c, const char *name, const uint16_t *data); /* borrowed */
int vxo_codec_init_synthetic(vxo_codec *c, uint64_t seed, float std);
/* stop: 0 concat input [T][292], 1 after_input_conv [T][1024],
 * 2+2s after_stage{s}_transformer, 3+2s after_stage{s}_conv_up (s < 3),
 * 9 audio [8T][240] (the names of debugCodecDecode, src/engine.ts:1719-1985) */
size_t vxo_codec_stop_count(int T, int stop);
int vxo_codec_decode(vxo_codec *c, const uint32_t *sem, const uint32_t *ac, int T, int stop,
                     float *out);
/* every intermediate k with outs[k] != NULL (outs[10]) in one pass */
int vxo_codec_decode_all(vxo_codec *c, const uint32_t *sem, const uint32_t *ac, int T,
                         float *const *outs);

#ifdef __cplusplus
}
#endif
#endif
