/*
 * vx_oracle_codec.c -- CPU restatement of the reference's codec decoder
 * (codes -> 24 kHz waveform): codecDecode, src/engine.ts:1402-1713, with the
 * codec shaders of src/shaders.ts:817-1110, 1432-1868.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker for the HIP codec decoder.
 * The product never links this file.
 *
 * Each kernel restates one WGSL shader with its f32 arithmetic and its
 * summation order (sequential loops where the shader loops in one thread,
 * 256 strided lane partials + tree where it reduces across a workgroup).
 * How each part is pinned (tests/test_oracle_codec.py):
 *   normalizeCodebook    numpy f32 division + float16 RNE; the eps clamp
 *   vqLookup / fsq       known answers (code 2 -> -1, 12 -> 0, 22 -> +1)
 *   causalConv1d         torch conv1d over a left-padded input with the
 *                        weight-norm weight g * v / ||v|| (f64)
 *   convTranspose (+scale) torch conv_transpose1d, right-trimmed, with the
 *                        per-input-channel weight norm (f64)
 *   qkNorm, rmsNorm      torch rms_norm per head / per frame (f64)
 *   windowed ALiBi attention  a dense f64 attention with an explicit
 *                        causal-window mask and bias
 *   whole decoder        a float64 torch model of the decoder written from
 *                        the architecture (tests/codec_f64.py), every
 *                        intermediate
 * Semantic codes >= 8192 index past the 8192-row codebook in the reference
 * (vqLookup has no bound check; WebGPU clamps such reads in an
 * implementation-defined way).  Here they read a zero row: parity unpinned
 * for those codes.  The WGSL builtins' bit-level behaviour (exp, pow, sqrt,
 * division, pack2x16float rounding) is parity unpinned, as in vx_oracle.c.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "vx_oracle.h"
#include "vx_oracle_internal.h"

#define WG 256

static const float *g_h;
static inline float H(uint16_t h) { return g_h[h]; }

/* codec constants, src/types.ts:98-122 */
enum {
  CD = 1024,     /* dim */
  CHID = 4096,   /* hidden_dim */
  CNH = 8,       /* n_heads */
  CHD = 128,     /* head_dim */
  CSEM = 8192,   /* semantic_codebook_size */
  CSEMD = 256,   /* semantic_dim */
  CNAC = 36,     /* n_acoustic_codebook */
  CLEV = 21,     /* acoustic_codebook_size */
  CIN = CSEMD + CNAC,
  CPATCH = 240,  /* patch_size */
  CSTAGES = 4,
  CLPS = 2       /* decoder_layers_per_stage */
};
static const float CNORM_EPS = 0.01f, CQK_EPS = 1e-6f;
/* codecDecode's per-stage tables, src/engine.ts:1505-1507 */
static const int kStageStride[4] = {2, 2, 2, 1};
static const int kStageKernel[4] = {4, 4, 4, 3};
static const int kWindow[4] = {2, 4, 8, 16};

/* ======================================================================= */
/* Kernels                                                                  */
/* ======================================================================= */

/* normalizeCodebook, src/shaders.ts:851-885 (engine: normalizeVQCodebook
 * :593-613): cb[i][d] = f16(f32(cb[i][d]) / max(f32(usage[i]), eps)) */
void vxo_normalize_codebook(const uint16_t *sum, const uint16_t *usage, uint16_t *out,
                            int n_entries, int dim, float eps) {
  g_h = vxo_i_h2f_table();
  for (int i = 0; i < n_entries; i++) {
    float u = H(usage[i]);
    u = u > eps ? u : eps;
    for (int d = 0; d < dim; d++)
      out[(size_t)i * dim + d] = vxo_f32_to_f16(H(sum[(size_t)i * dim + d]) / u);
  }
}

/* vqLookup, src/shaders.ts:817-845; rows >= n_entries read as zero */
void vxo_vq_lookup(const uint32_t *codes, const uint16_t *cb, float *out, int T, int dim,
                   int n_entries) {
  g_h = vxo_i_h2f_table();
  for (int t = 0; t < T; t++)
    for (int d = 0; d < dim; d++)
      out[(size_t)t * dim + d] =
          codes[t] < (uint32_t)n_entries ? H(cb[(size_t)codes[t] * dim + d]) : 0.0f;
}

/* fsqDequant, src/shaders.ts:891-914: f32(code - offset) * 2 / (levels - 1) - 1
 * with u32 wrap-around of code - offset */
void vxo_fsq_dequant(const uint32_t *codes, float *out, int n, int levels, int offset) {
  for (int i = 0; i < n; i++) {
    uint32_t c = codes[i] - (uint32_t)offset;
    out[i] = (float)c * 2.0f / (float)(levels - 1) - 1.0f;
  }
}

/* causalConv1d, src/shaders.ts:927-985.  input [n_frames*stride][c_in],
 * weight [c_out][c_in][kernel], g [c_out]; output [n_frames][c_out]. */
void vxo_causal_conv1d(const float *in, const uint16_t *w, const uint16_t *g, float *out,
                       int c_in, int c_out, int kernel, int n_frames, int stride) {
  g_h = vxo_i_h2f_table();
  const int pad = kernel - 1, n_in = n_frames * stride;
#pragma omp parallel for schedule(static)
  for (int co = 0; co < c_out; co++) {
    const float gv = H(g[co]);
    const uint16_t *wr = w + (size_t)co * c_in * kernel;
    float wn = 0.0f;
    for (int p = 0; p < c_in * kernel / 2; p++) {
      float a = H(wr[2 * p]), b = H(wr[2 * p + 1]);
      wn += a * a + b * b;
    }
    wn = 1.0f / sqrtf(wn + 1e-12f);
    for (int t = 0; t < n_frames; t++) {
      float sum = 0.0f;
      for (int ci = 0; ci < c_in; ci++)
        for (int k = 0; k < kernel; k++) {
          int ti = t * stride - pad + k;
          if (ti >= 0 && ti < n_in) {
            float wv = H(wr[(size_t)ci * kernel + k]);
            sum += (wv * wn * gv) * in[(size_t)ti * c_in + ci];
          }
        }
      out[(size_t)t * c_out + co] = sum;
    }
  }
}

/* convTransposeNormScale, src/shaders.ts:1009-1058 (engine:
 * precomputeConvTransposeScales :621-657): scale[ci] = g[ci] / ||w[ci,:,:]||
 * with the 256-lane strided sum + tree */
void vxo_conv_transpose_scale(const uint16_t *w, const uint16_t *g, float *scale, int c_in,
                              int c_out, int kernel) {
  g_h = vxo_i_h2f_table();
  const int n = c_out * kernel;
#pragma omp parallel for schedule(static)
  for (int ci = 0; ci < c_in; ci++) {
    float sd[WG];
    const uint16_t *wr = w + (size_t)ci * n;
    for (int t = 0; t < WG; t++) {
      float ss = 0.0f;
      for (int i = t; i < n; i += WG) {
        float v = H(wr[i]);
        ss += v * v;
      }
      sd[t] = ss;
    }
    float tot = vxo_i_tree_sum(sd);
    scale[ci] = H(g[ci]) * (1.0f / sqrtf(tot + 1e-12f));
  }
}

/* causalConvTranspose1d, src/shaders.ts:1066-1110.  input [n_out/stride][c_in],
 * weight [c_in][c_out][kernel]; output [n_out][c_out]. */
void vxo_conv_transpose1d(const float *in, const uint16_t *w, const float *scale, float *out,
                          int c_in, int c_out, int kernel, int n_out, int stride) {
  g_h = vxo_i_h2f_table();
  const int n_in = n_out / stride;
#pragma omp parallel for schedule(static)
  for (int co = 0; co < c_out; co++)
    for (int t = 0; t < n_out; t++) {
      float sum = 0.0f;
      for (int k = 0; k < kernel; k++) {
        int diff = t - k;
        if (diff >= 0 && diff % stride == 0) {
          int ti = diff / stride;
          if (ti < n_in)
            for (int ci = 0; ci < c_in; ci++) {
              float wv = H(w[((size_t)ci * c_out + co) * kernel + k]);
              sum += (wv * scale[ci]) * in[(size_t)ti * c_in + ci];
            }
        }
      }
      out[(size_t)t * c_out + co] = sum;
    }
}

/* batchedRmsNorm, src/shaders.ts:1646-1692 */
void vxo_batched_rmsnorm(const float *in, const uint16_t *w, float *out, int dim, int T,
                         float eps) {
  g_h = vxo_i_h2f_table();
  for (int t = 0; t < T; t++) {
    const float *x = in + (size_t)t * dim;
    float sd[WG];
    for (int l = 0; l < WG; l++) {
      float ss = 0.0f;
      for (int i = l; i < dim; i += WG) ss += x[i] * x[i];
      sd[l] = ss;
    }
    float rms = 1.0f / sqrtf(vxo_i_tree_sum(sd) / (float)dim + eps);
    for (int i = 0; i < dim; i++) out[(size_t)t * dim + i] = x[i] * rms * H(w[i]);
  }
}

/* batchedMatvecF16, src/shaders.ts:1591-1640: out[t][m] = A[m,:] . in[t] */
void vxo_batched_matvec_f16(const uint16_t *A, const float *in, float *out, int M, int K,
                            int T) {
  for (int t0 = 0; t0 < T; t0 += 8) {
    const int nb = T - t0 < 8 ? T - t0 : 8;
    const float *xs[8];
    float *ys[8];
    for (int b = 0; b < nb; b++) {
      xs[b] = in + (size_t)(t0 + b) * K;
      ys[b] = out + (size_t)(t0 + b) * M;
    }
    vxo_i_matvec_multi(A, xs, ys, nb, M, K);
  }
}

/* qkNorm, src/shaders.ts:1787-1830: per (frame, head) RMS over head_dim,
 * weight [n_heads * head_dim] read at h * head_dim */
void vxo_qk_norm(float *data, const uint16_t *w, int n_heads, int head_dim, int T, float eps) {
  g_h = vxo_i_h2f_table();
  for (int idx = 0; idx < T * n_heads; idx++) {
    float *x = data + (size_t)idx * head_dim;
    const int h = idx % n_heads;
    float ss = 0.0f;
    for (int d = 0; d < head_dim; d++) ss += x[d] * x[d];
    float rms = 1.0f / sqrtf(ss / (float)head_dim + eps);
    for (int d = 0; d < head_dim; d++) x[d] = x[d] * rms * H(w[h * head_dim + d]);
  }
}

/* alibiAttnScore + codecSoftmax + codecAttnValue, src/shaders.ts:1432-1585:
 * q, k, v, out [T][n_heads][head_dim]; keys ki in [max(0, qi-W+1), qi] */
void vxo_codec_attention(const float *q, const float *k, const float *v, float *out,
                         int n_heads, int head_dim, int T, int W) {
  const int nhd = n_heads * head_dim;
  const float scale = 1.0f / sqrtf((float)head_dim);
#pragma omp parallel for schedule(static)
  for (int qi = 0; qi < T; qi++) {
    float sc[64];
    for (int h = 0; h < n_heads; h++) {
      const int k0 = qi + 1 > W ? qi - W + 1 : 0;
      const float slope = powf(2.0f, -8.0f * (float)(h + 1) / (float)n_heads);
      for (int s = 0; s < W; s++) {
        const int ki = k0 + s;
        if (ki > qi) {
          sc[s] = -1e30f;
          continue;
        }
        const float alibi = -slope * (float)(qi - ki);
        float dot = 0.0f;
        const float *qq = q + (size_t)qi * nhd + h * head_dim;
        const float *kk = k + (size_t)ki * nhd + h * head_dim;
        for (int d = 0; d < head_dim; d++) dot += qq[d] * kk[d];
        sc[s] = dot * scale + alibi;
      }
      float mx = -1e30f;
      for (int s = 0; s < W; s++) mx = fmaxf(mx, sc[s]);
      float es = 0.0f;
      for (int s = 0; s < W; s++) {
        sc[s] = expf(sc[s] - mx);
        es += sc[s];
      }
      for (int s = 0; s < W; s++) sc[s] /= es;
      for (int d = 0; d < head_dim; d++) {
        float sum = 0.0f;
        for (int s = 0; s < W; s++) {
          const int ki = k0 + s;
          if (ki > qi) break;
          sum += sc[s] * v[(size_t)ki * nhd + h * head_dim + d];
        }
        out[(size_t)qi * nhd + h * head_dim + d] = sum;
      }
    }
  }
}

/* ======================================================================= */
/* Weights (src/engine.ts:700-770)                                          */
/* ======================================================================= */

typedef struct {
  const uint16_t *attn_norm, *q_norm, *k_norm, *wq, *wk, *wv, *wo, *attn_scale, *ffn_norm, *w1,
      *w2, *w3, *ffn_scale;
} cx_layer;

typedef struct {
  char name[112];
  const uint16_t **slot;
  size_t numel;
  float mean; /* synthetic initialisation: 1 for gains and scales */
} cx_slot;

struct vxo_codec {
  const uint16_t *in_w, *in_g, *out_w, *out_g, *cb_sum, *cb_usage;
  const uint16_t *up_w[3], *up_g[3];
  cx_layer L[CSTAGES][CLPS];
  cx_slot slots[160];
  int n_slots;
  uint16_t *owned[160];
  int n_owned;
};

static void cx_add(vxo_codec *c, const char *name, const uint16_t **slot, size_t numel,
                   float mean) {
  cx_slot *s = &c->slots[c->n_slots++];
  snprintf(s->name, sizeof s->name, "%s", name);
  s->slot = slot;
  s->numel = numel;
  s->mean = mean;
}

vxo_codec *vxo_codec_create(void) {
  vxo_codec *c = (vxo_codec *)calloc(1, sizeof(vxo_codec));
  const char *P = "audio_tokenizer.";
  char nm[112];
#define ADD(field, n, mean, ...)                      \
  do {                                                \
    snprintf(nm, sizeof nm, __VA_ARGS__);             \
    cx_add(c, nm, &(field), (size_t)(n), (mean));     \
  } while (0)
  ADD(c->in_w, (size_t)CD * CIN * 3, 0.f, "%sdecoder_blocks.0.conv.parametrizations.weight.original1", P);
  ADD(c->in_g, CD, 1.f, "%sdecoder_blocks.0.conv.parametrizations.weight.original0", P);
  for (int s = 0; s < CSTAGES; s++) {
    for (int l = 0; l < CLPS; l++) {
      cx_layer *L = &c->L[s][l];
      const int b = 1 + 2 * s;
#define LW(field, n, mean, suffix) \
  ADD(L->field, n, mean, "%sdecoder_blocks.%d.layers.%d.%s", P, b, l, suffix)
      LW(attn_norm, CD, 1.f, "attention_norm.weight");
      LW(q_norm, CD, 1.f, "attention.q_norm.weight");
      LW(k_norm, CD, 1.f, "attention.k_norm.weight");
      LW(wq, (size_t)CD * CD, 0.f, "attention.wq.weight");
      LW(wk, (size_t)CD * CD, 0.f, "attention.wk.weight");
      LW(wv, (size_t)CD * CD, 0.f, "attention.wv.weight");
      LW(wo, (size_t)CD * CD, 0.f, "attention.wo.weight");
      LW(attn_scale, CD, 1.f, "attention_scale");
      LW(ffn_norm, CD, 1.f, "ffn_norm.weight");
      LW(w1, (size_t)CHID * CD, 0.f, "feed_forward.w1.weight");
      LW(w2, (size_t)CD * CHID, 0.f, "feed_forward.w2.weight");
      LW(w3, (size_t)CHID * CD, 0.f, "feed_forward.w3.weight");
      LW(ffn_scale, CD, 1.f, "ffn_scale");
#undef LW
    }
    if (s < 3) {
      ADD(c->up_w[s], (size_t)CD * CD * 4, 0.f,
          "%sdecoder_blocks.%d.conv.parametrizations.weight.original1", P, 2 + 2 * s);
      ADD(c->up_g[s], CD, 1.f, "%sdecoder_blocks.%d.conv.parametrizations.weight.original0", P,
          2 + 2 * s);
    }
  }
  ADD(c->out_w, (size_t)CPATCH * CD * 7, 0.f, "%soutput_proj.conv.parametrizations.weight.original1", P);
  ADD(c->out_g, CPATCH, 1.f, "%soutput_proj.conv.parametrizations.weight.original0", P);
  ADD(c->cb_sum, (size_t)CSEM * CSEMD, 0.f, "%squantizer.semantic_codebook.embedding_sum", P);
  ADD(c->cb_usage, CSEM, 1.f, "%squantizer.semantic_codebook.cluster_usage", P);
#undef ADD
  return c;
}

void vxo_codec_destroy(vxo_codec *c) {
  if (!c) return;
  for (int i = 0; i < c->n_owned; i++) free(c->owned[i]);
  free(c);
}

static cx_slot *cx_find(const vxo_codec *c, const char *name) {
  for (int i = 0; i < c->n_slots; i++)
    if (!strcmp(c->slots[i].name, name)) return (cx_slot *)&c->slots[i];
  return NULL;
}

int vxo_codec_n_weights(const vxo_codec *c) { return c->n_slots; }
const char *vxo_codec_weight_name(const vxo_codec *c, int i) {
  return i >= 0 && i < c->n_slots ? c->slots[i].name : NULL;
}
size_t vxo_codec_weight_numel(const vxo_codec *c, const char *name) {
  cx_slot *s = cx_find(c, name);
  return s ? s->numel : 0;
}
const uint16_t *vxo_codec_weight(const vxo_codec *c, const char *name) {
  cx_slot *s = cx_find(c, name);
  return s ? *s->slot : NULL;
}
int vxo_codec_set_weight(vxo_codec *c, const char *name, const uint16_t *data) {
  cx_slot *s = cx_find(c, name);
  if (!s) return -1;
  *s->slot = data;
  return 0;
}

int vxo_codec_init_synthetic(vxo_codec *c, uint64_t seed, float std) {
  for (int i = 0; i < c->n_slots; i++) {
    cx_slot *s = &c->slots[i];
    uint16_t *buf = (uint16_t *)malloc(s->numel * sizeof(uint16_t));
    if (!buf) return -1;
    vxo_gen_f16(seed, vxo_name_stream(s->name), s->numel, s->mean, std, buf);
    c->owned[c->n_owned++] = buf;
    *s->slot = buf;
  }
  return 0;
}

/* ======================================================================= */
/* codecDecode / debugCodecDecode (src/engine.ts:1402-1985)                 */
/* ======================================================================= */

/* frames at a stop point: 0 concat [T][292], 1 after_input_conv,
 * 2 + 2s after_stage{s}_transformer, 3 + 2s after_stage{s}_conv_up (s < 3),
 * 9 audio [8T][240] */
static int stop_frames(int T, int stop) {
  if (stop <= 2) return T;
  if (stop == 9) return 8 * T;
  const int s = (stop - 2) / 2, up = (stop - 2) % 2;
  return T << (s + up);
}

size_t vxo_codec_stop_count(int T, int stop) {
  if (stop < 0 || stop > 9 || T < 0) return 0;
  const size_t f = (size_t)stop_frames(T, stop);
  return f * (stop == 0 ? CIN : stop == 9 ? CPATCH : CD);
}

static float *fa(size_t n) {
  float *p = (float *)calloc(n ? n : 1, sizeof(float));
  if (!p) {
    fprintf(stderr, "vx_oracle_codec: out of memory\n");
    abort();
  }
  return p;
}

/* codecDecode with every debugCodecDecode intermediate whose outs[k] is set
 * (outs[10], entries nullable); stops after the last one requested */
int vxo_codec_decode_all(vxo_codec *c, const uint32_t *sem, const uint32_t *ac, int T,
                         float *const *outs) {
  int last = -1;
  for (int k = 0; k < 10; k++)
    if (outs[k]) last = k;
  if (T < 1 || last < 0) return -1;
  for (int i = 0; i < c->n_slots; i++)
    if (!*c->slots[i].slot) return -2;
  g_h = vxo_i_h2f_table();
  const int Tmax = 8 * T;
  /* normalizeVQCodebook at load, src/engine.ts:593-613 */
  uint16_t *cb = (uint16_t *)malloc((size_t)CSEM * CSEMD * 2);
  vxo_normalize_codebook(c->cb_sum, c->cb_usage, cb, CSEM, CSEMD, 1e-5f);
  float *sem_e = fa((size_t)T * CSEMD), *ac_f = fa((size_t)T * CNAC), *cat = fa((size_t)T * CIN);
  vxo_vq_lookup(sem, cb, sem_e, T, CSEMD, CSEM);
  vxo_fsq_dequant(ac, ac_f, T * CNAC, CLEV, 2);
  for (int t = 0; t < T; t++) {
    memcpy(cat + (size_t)t * CIN, sem_e + (size_t)t * CSEMD, CSEMD * 4);
    memcpy(cat + (size_t)t * CIN + CSEMD, ac_f + (size_t)t * CNAC, CNAC * 4);
  }
  free(cb);
  free(sem_e);
  free(ac_f);
  if (outs[0]) memcpy(outs[0], cat, (size_t)T * CIN * 4);
  if (last == 0) {
    free(cat);
    return 0;
  }
  float *cur = fa((size_t)Tmax * CD), *res = fa((size_t)Tmax * CD), *xn = fa((size_t)Tmax * CD),
        *q = fa((size_t)Tmax * CD), *k = fa((size_t)Tmax * CD), *v = fa((size_t)Tmax * CD),
        *ao = fa((size_t)Tmax * CD), *o = fa((size_t)Tmax * CD), *gate = fa((size_t)Tmax * CHID),
        *up = fa((size_t)Tmax * CHID), *nxt = fa((size_t)Tmax * CD);
  vxo_causal_conv1d(cat, c->in_w, c->in_g, cur, CIN, CD, 3, T, 1);
  free(cat);
  int curT = T, at = 1;
#define EMIT()                                                          \
  do {                                                                  \
    if (outs[at]) memcpy(outs[at], cur, (size_t)curT * CD * 4);         \
    if (at == last) goto cleanup;                                       \
  } while (0)
  EMIT();
  for (int s = 0; s < CSTAGES; s++) {
    for (int l = 0; l < CLPS; l++) {
      const cx_layer *L = &c->L[s][l];
      const size_t n = (size_t)curT * CD;
      memcpy(res, cur, n * 4);
      vxo_batched_rmsnorm(cur, L->attn_norm, xn, CD, curT, CNORM_EPS);
      vxo_batched_matvec_f16(L->wq, xn, q, CD, CD, curT);
      vxo_batched_matvec_f16(L->wk, xn, k, CD, CD, curT);
      vxo_batched_matvec_f16(L->wv, xn, v, CD, CD, curT);
      vxo_qk_norm(q, L->q_norm, CNH, CHD, curT, CQK_EPS);
      vxo_qk_norm(k, L->k_norm, CNH, CHD, curT, CQK_EPS);
      vxo_codec_attention(q, k, v, ao, CNH, CHD, curT, kWindow[s]);
      vxo_batched_matvec_f16(L->wo, ao, o, CD, CD, curT);
      for (size_t i = 0; i < n; i++) cur[i] = o[i] * H(L->attn_scale[i % CD]) + res[i];
      memcpy(res, cur, n * 4);
      vxo_batched_rmsnorm(cur, L->ffn_norm, xn, CD, curT, CNORM_EPS);
      vxo_batched_matvec_f16(L->w1, xn, gate, CHID, CD, curT);
      vxo_batched_matvec_f16(L->w3, xn, up, CHID, CD, curT);
      for (size_t i = 0; i < (size_t)curT * CHID; i++) {
        const float g = gate[i];
        gate[i] = g / (1.0f + expf(-g)) * up[i];
      }
      vxo_batched_matvec_f16(L->w2, gate, o, CD, CHID, curT);
      for (size_t i = 0; i < n; i++) cur[i] = o[i] * H(L->ffn_scale[i % CD]) + res[i];
    }
    at = 2 + 2 * s;
    EMIT();
    if (kStageStride[s] > 1) {
      float scale[CD];
      vxo_conv_transpose_scale(c->up_w[s], c->up_g[s], scale, CD, CD, kStageKernel[s]);
      const int newT = curT * kStageStride[s];
      vxo_conv_transpose1d(cur, c->up_w[s], scale, nxt, CD, CD, kStageKernel[s], newT,
                           kStageStride[s]);
      float *tmp = cur;
      cur = nxt;
      nxt = tmp;
      curT = newT;
      at = 3 + 2 * s;
      EMIT();
    }
  }
#undef EMIT
  vxo_causal_conv1d(cur, c->out_w, c->out_g, outs[9], CD, CPATCH, 7, curT, 1);
cleanup:;
  float *bufs[] = {cur, res, xn, q, k, v, ao, o, gate, up, nxt};
  for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; i++) free(bufs[i]);
  return 0;
}

int vxo_codec_decode(vxo_codec *c, const uint32_t *sem, const uint32_t *ac, int T, int stop,
                     float *out) {
  if (stop < 0 || stop > 9 || !out) return -1;
  float *outs[10] = {0};
  outs[stop] = out;
  return vxo_codec_decode_all(c, sem, ac, T, outs);
}
