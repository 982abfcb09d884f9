/*
 * vx_oracle.c -- CPU restatement of the reference Voxtral frame loop.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker and the CPU baseline.  The
 * product never links this file.  Build: oracle/Makefile (gcc, OpenMP,
 * -ffp-contract=off so no product is fused into an FMA that the WGSL source
 * does not ask for).
 *
 * How each part is pinned (checked by tests/test_oracle_*.py):
 *   f16 conversion        exhaustive round trip of all 65536 halves; numpy
 *                         float16 RNE on 10^6 random floats and edge cases
 *   splitmix64            published first outputs of the state-0 stream
 *   normal generator      exact integer Irwin-Hall sum recomputed in numpy;
 *                         moments; bit-identity with the GPU generator
 *   FM noise (vxo_gauss)  Python restatement with exact fma, bit for bit;
 *                         numpy Box-Muller in f64; moments and tails;
 *                         bit-identity with the GPU generator
 *   matvec_f16            f64 numpy product (tolerance), and an explicit
 *                         restatement of the 256-lane strided/tree order
 *   rmsnorm               torch.nn.functional.rms_norm (f64)
 *   rope                  closed form; identity at pos 0; norm preservation
 *   attention             torch scaled_dot_product_attention with GQA
 *                         repeat_interleave (f64); softmax sums to 1;
 *                         identical keys give the mean of V
 *   swiglu                torch.nn.functional.silu (f64)
 *   time embedding        closed form in f64
 *   cfg / euler           closed forms; v_c == v_u gives v; v = 0 is a no-op
 *   fsq                   known answers -1 -> 2, 0 -> 12, +1 -> 22, ties to
 *                         even, clamping
 *   argmax                numpy argmax on tie-free data; exact ties against
 *                         a hand trace of the 256-lane tree rule
 *   multi-codebook embed  row formula 8194 + k*23 + code, f64 sum
 *   bi-attention          torch SDPA over 3 tokens (f64)
 *   backbone step         a float64 numpy transformer layer written from the
 *                         model definition (tests/oracle_np.py)
 *   fm forward            the same numpy model over the Euler/CFG loop; and
 *                         per-position vs batched dataflow bit-identity
 * The WGSL builtins' bit-level behaviour inside a browser's WebGPU
 * implementation (exp, pow, sin, cos, sqrt, division, FMA contraction) is
 * parity unpinned: no WebGPU runtime exists here and the reference ships no
 * golden vectors.  This file uses correctly rounded libm-style calls.
 */
#include "vx_oracle.h"
#include "vx_oracle_internal.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define WG 256 /* workgroup size of every reduction shader, src/shaders.ts:32 */

/* ======================================================================= */
/* Numbers                                                                  */
/* ======================================================================= */

static float g_h2f[65536];
static int g_h2f_ready = 0;

static float h2f_slow(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t exp = (h >> 10) & 0x1f;
  uint32_t man = h & 0x3ff;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: normalise */
      int e = -1;
      do {
        man <<= 1;
        e++;
      } while ((man & 0x400) == 0);
      man &= 0x3ff;
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

static void h2f_init(void) {
  if (g_h2f_ready) return;
  for (uint32_t i = 0; i < 65536; i++) g_h2f[i] = h2f_slow((uint16_t)i);
  g_h2f_ready = 1;
}

float vxo_f16_to_f32(uint16_t h) {
  h2f_init();
  return g_h2f[h];
}

static inline float H(uint16_t h) { return g_h2f[h]; }

uint16_t vxo_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) { /* inf or nan */
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ff));
    return (uint16_t)(sign | 0x7c00u);
  }
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to inf */
  if (ax < 0x38800000u) { /* below the smallest normal half: 2^-14 */
    if (ax <= 0x33000000u) return (uint16_t)sign; /* <= 2^-25: rounds to 0 */
    /* Subnormal half q * 2^-24.  The float is m * 2^(e-150) with a 24-bit
     * significand m, i.e. m * 2^(e-126) units of 2^-24; e <= 112, so the
     * significand is shifted right by rsh = 126 - e (14..24) bits, RNE.
     * q == 1024 correctly becomes the smallest normal (0x0400). */
    uint32_t e = ax >> 23;
    uint32_t m = (ax & 0x7fffff) | 0x800000;
    int rsh = 126 - (int)e;
    uint32_t q = m >> rsh;
    uint32_t rem = m & ((1u << rsh) - 1);
    uint32_t half = 1u << (rsh - 1);
    if (rem > half || (rem == half && (q & 1))) q++;
    return (uint16_t)(sign | q);
  }
  /* normal half */
  uint32_t e = (ax >> 23) - 127 + 15;
  uint32_t m = ax & 0x7fffff;
  uint32_t q = (e << 10) | (m >> 13);
  uint32_t rem = m & 0x1fff;
  if (rem > 0x1000 || (rem == 0x1000 && (q & 1))) q++;
  return (uint16_t)(sign | q);
}

static const uint64_t GOLDEN = 0x9E3779B97F4A7C15ull;

static inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

uint64_t vxo_splitmix64_next(uint64_t *state) {
  *state += GOLDEN;
  return mix64(*state);
}

uint64_t vxo_name_stream(const char *name) {
  uint64_t h = 0xcbf29ce484222325ull;
  for (const unsigned char *p = (const unsigned char *)name; *p; p++) {
    h ^= *p;
    h *= 0x100000001b3ull;
  }
  return h;
}

float vxo_normal(uint64_t seed, uint64_t stream, uint64_t idx) {
  uint64_t s0 = mix64(seed) ^ stream;
  int64_t s = 0;
  for (uint64_t j = 0; j < 4; j++) {
    uint64_t h = mix64(s0 + (4 * idx + j + 1) * GOLDEN);
    s += (int64_t)(h & 0xFFFFF);
    s += (int64_t)((h >> 20) & 0xFFFFF);
    s += (int64_t)((h >> 40) & 0xFFFFF);
  }
  int64_t zi = s - 6 * (int64_t)0xFFFFF;
  return (float)zi * 0x1p-20f;
}

/* Gaussian of (seed, stream, idx) by the Box-Muller transform the reference
 * uses for the FM noise (src/engine.ts:1264-1273: sqrt(-2 ln u1) cos(2 pi u2),
 * u1, u2 uniform), from two counter-hashed uniforms: u1 = N 2^-53 in (0, 1]
 * with N = (h1 >> 11) + 1, u2 = U 2^-53 in [0, 1) with U = h2 >> 11.  The
 * logarithm and cosine are evaluated with IEEE double additions,
 * multiplications, one division, one square root and explicit fused
 * multiply-adds in a fixed order (no library transcendental), so the device
 * generator gives the identical float:
 *   ln u1 = (e - 53) ln 2 + ln m, N = m 2^e with m in [sqrt(1/2), sqrt(2)),
 *           ln m = 2 (s + s^3 p(s^2)), s = (m - 1) / (m + 1), p the atanh
 *           series 1/3 + s^2/5 + ... + s^14/17 (Horner);
 *   cos(2 pi u2): quadrant q = U >> 51, x = (U mod 2^51) 2^-51 (pi/2),
 *           cos x, sin x by their Taylor series to x^20 / x^21 (Horner),
 *           then cos x, -sin x, -cos x, sin x for q = 0..3. */
static const double BM_LOGC[8] = {0x1.5555555555555p-2, 0x1.999999999999ap-3, 0x1.2492492492492p-3,
                                  0x1.c71c71c71c71cp-4, 0x1.745d1745d1746p-4, 0x1.3b13b13b13b14p-4,
                                  0x1.1111111111111p-4, 0x1.e1e1e1e1e1e1ep-5};
static const double BM_COSC[10] = {-0x1.0000000000000p-1, 0x1.5555555555555p-5,  -0x1.6c16c16c16c17p-10,
                                   0x1.a01a01a01a01ap-16, -0x1.27e4fb7789f5cp-22, 0x1.1eed8eff8d898p-29,
                                   -0x1.93974a8c07c9dp-37, 0x1.ae7f3e733b81fp-45, -0x1.6827863b97d97p-53,
                                   0x1.e542ba4020225p-62};
static const double BM_SINC[10] = {-0x1.5555555555555p-3, 0x1.1111111111111p-7,  -0x1.a01a01a01a01ap-13,
                                   0x1.71de3a556c734p-19, -0x1.ae64567f544e4p-26, 0x1.6124613a86d09p-33,
                                   -0x1.ae7f3e733b81fp-41, 0x1.952c77030ad4ap-49, -0x1.2f49b46814157p-57,
                                   0x1.71b8ef6dcf572p-66};
#define BM_LN2 0x1.62e42fefa39efp-1
#define BM_PIO2 0x1.921fb54442d18p+0
#define BM_SQRT2 0x1.6a09e667f3bcdp+0

float vxo_gauss(uint64_t seed, uint64_t stream, uint64_t idx) {
  const uint64_t s0 = mix64(seed) ^ stream;
  const uint64_t h1 = mix64(s0 + (2 * idx + 1) * GOLDEN), h2 = mix64(s0 + (2 * idx + 2) * GOLDEN);
  const double d = (double)((h1 >> 11) + 1); /* exact */
  uint64_t bits;
  memcpy(&bits, &d, 8);
  int e = (int)((bits >> 52) & 0x7FF) - 1023;
  const uint64_t mb = (bits & 0xFFFFFFFFFFFFFull) | 0x3FF0000000000000ull;
  double m;
  memcpy(&m, &mb, 8);
  if (m > BM_SQRT2) {
    m = m * 0.5;
    e += 1;
  }
  const double s = (m - 1.0) / (m + 1.0), s2 = s * s;
  double p = BM_LOGC[7];
  for (int k = 6; k >= 0; k--) p = fma(s2, p, BM_LOGC[k]);
  const double lm = 2.0 * fma(s * s2, p, s);
  const double lu = fma((double)(e - 53), BM_LN2, lm);
  const double r = sqrt(-2.0 * lu);
  const uint64_t U = h2 >> 11;
  const int q = (int)(U >> 51);
  const double x = ((double)(U & ((1ull << 51) - 1)) * 0x1p-51) * BM_PIO2, x2 = x * x;
  double c = BM_COSC[9], sn = BM_SINC[9];
  for (int k = 8; k >= 0; k--) {
    c = fma(x2, c, BM_COSC[k]);
    sn = fma(x2, sn, BM_SINC[k]);
  }
  c = fma(x2, c, 1.0);
  sn = fma(x * x2, sn, x);
  const double cs = q == 0 ? c : q == 1 ? -sn : q == 2 ? -c : sn;
  return (float)(r * cs);
}

void vxo_gen_gauss_f32(uint64_t seed, uint64_t stream, size_t n, float *out) {
  for (size_t i = 0; i < n; i++) out[i] = vxo_gauss(seed, stream, (uint64_t)i);
}

void vxo_gen_f32(uint64_t seed, uint64_t stream, size_t n, float mean,
                 float std, float *out) {
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < (long long)n; i++) {
    float t = vxo_normal(seed, stream, (uint64_t)i) * std;
    out[i] = mean + t;
  }
}

void vxo_gen_f16(uint64_t seed, uint64_t stream, size_t n, float mean,
                 float std, uint16_t *out) {
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < (long long)n; i++) {
    float t = vxo_normal(seed, stream, (uint64_t)i) * std;
    out[i] = vxo_f32_to_f16(mean + t);
  }
}

/* ======================================================================= */
/* Kernels (src/shaders.ts)                                                 */
/* ======================================================================= */

/* Shared-memory tree of the reduction shaders:
 * for s = 128..1: sdata[tid] += sdata[tid + s]  (e.g. src/shaders.ts:59-64) */
static inline float tree_sum(float *sd) {
  for (int s = WG / 2; s > 0; s >>= 1)
    for (int t = 0; t < s; t++) sd[t] += sd[t + s];
  return sd[0];
}

/* One matvecF16 workgroup (src/shaders.ts:21-71) for `nb` input vectors that
 * share the weight row: lane tid sums pairs pk = tid, tid+256, ...; each pair
 * contributes (a0*x0 + a1*x1); then the tree.  xs[b] points at vector b. */
static void matvec_row(const uint16_t *row, const float *const *xs, int nb,
                       int K, float *out /* [nb] */) {
  const int Kp = K / 2;
  float rowf[2 * WG];
  float part[8][WG];
  for (int b = 0; b < nb; b++) memset(part[b], 0, sizeof(part[b]));
  for (int base = 0; base < Kp; base += WG) {
    int n = Kp - base < WG ? Kp - base : WG;
    for (int t = 0; t < 2 * n; t++) rowf[t] = H(row[2 * base + t]);
    for (int b = 0; b < nb; b++) {
      const float *x = xs[b] + 2 * base;
      float *p = part[b];
      for (int t = 0; t < n; t++) {
        float s0 = rowf[2 * t] * x[2 * t];
        float s1 = rowf[2 * t + 1] * x[2 * t + 1];
        p[t] += s0 + s1;
      }
    }
  }
  for (int b = 0; b < nb; b++) out[b] = tree_sum(part[b]);
}

void vxo_matvec_f16(const uint16_t *A, const float *x, float *y, int M, int K) {
  h2f_init();
#pragma omp parallel for schedule(static)
  for (int m = 0; m < M; m++) {
    const float *xs[1] = {x};
    matvec_row(A + (size_t)m * K, xs, 1, K, &y[m]);
  }
}

/* Batched form: ys[b][m] = A[m,:] . xs[b], same per-element arithmetic. */
static void matvec_f16_multi(const uint16_t *A, const float *const *xs,
                             float *const *ys, int nb, int M, int K) {
  h2f_init();
#pragma omp parallel for schedule(static)
  for (int m = 0; m < M; m++) {
    float out[8];
    matvec_row(A + (size_t)m * K, xs, nb, K, out);
    for (int b = 0; b < nb; b++) ys[b][m] = out[b];
  }
}

/* shared with vx_oracle_codec.c (vx_oracle_internal.h) */
const float *vxo_i_h2f_table(void) {
  h2f_init();
  return g_h2f;
}
float vxo_i_tree_sum(float *sd) { return tree_sum(sd); }
void vxo_i_matvec_multi(const uint16_t *A, const float *const *xs, float *const *ys, int nb,
                        int M, int K) {
  matvec_f16_multi(A, xs, ys, nb, M, K);
}

/* rmsNorm / rmsNormOffset, src/shaders.ts:137-183, 1278-1324 */
void vxo_rmsnorm(const float *x, const uint16_t *w, float *y, int dim, float eps) {
  h2f_init();
  float sd[WG];
  for (int t = 0; t < WG; t++) {
    float ss = 0.0f;
    for (int i = t; i < dim; i += WG) {
      float v = x[i];
      ss += v * v;
    }
    sd[t] = ss;
  }
  float total = tree_sum(sd);
  float rms = 1.0f / sqrtf(total / (float)dim + eps);
  for (int i = 0; i < dim; i++) y[i] = x[i] * rms * H(w[i]);
}

/* embeddingLookup, src/shaders.ts:193-213 */
void vxo_embedding(const uint16_t *table, int token, int dim, float *out) {
  h2f_init();
  for (int i = 0; i < dim; i++) out[i] = H(table[(size_t)token * dim + i]);
}

/* rope, src/shaders.ts:224-256: interleaved pairs (2i, 2i+1),
 * freq = 1/theta^(2i/dim), angle = pos * freq. */
void vxo_rope(float *qk, int head_dim, int pos, int n_heads, float theta) {
  int half = head_dim / 2;
  for (int idx = 0; idx < n_heads * half; idx++) {
    int head = idx / half, pair = idx % half;
    float freq = 1.0f / powf(theta, (float)(pair * 2) / (float)head_dim);
    float angle = (float)pos * freq;
    float c = cosf(angle), s = sinf(angle);
    int base = head * head_dim + pair * 2;
    float x0 = qk[base], x1 = qk[base + 1];
    qk[base] = x0 * c - x1 * s;
    qk[base + 1] = x0 * s + x1 * c;
  }
}

/* attnScore, src/shaders.ts:306-342 (cache layout [pos][kv_heads*head_dim]) */
void vxo_attn_scores(const float *q, const float *kcache, float *scores,
                     int n_heads, int n_kv_heads, int head_dim, int seq_len) {
  int rep = n_heads / n_kv_heads;
  float scale = 1.0f / sqrtf((float)head_dim);
  for (int h = 0; h < n_heads; h++) {
    int kvh = h / rep;
    for (int p = 0; p < seq_len; p++) {
      const float *qq = q + h * head_dim;
      const float *kk = kcache + (size_t)p * n_kv_heads * head_dim + kvh * head_dim;
      float dot = 0.0f;
      for (int d = 0; d < head_dim; d++) dot += qq[d] * kk[d];
      scores[h * seq_len + p] = dot * scale;
    }
  }
}

/* softmax, src/shaders.ts:348-409 */
void vxo_softmax(float *scores, int n_heads, int seq_len) {
  float sd[WG];
  for (int h = 0; h < n_heads; h++) {
    float *s = scores + (size_t)h * seq_len;
    for (int t = 0; t < WG; t++) {
      float m = -1e30f;
      for (int i = t; i < seq_len; i += WG) m = fmaxf(m, s[i]);
      sd[t] = m;
    }
    for (int st = WG / 2; st > 0; st >>= 1)
      for (int t = 0; t < st; t++) sd[t] = fmaxf(sd[t], sd[t + st]);
    float gmax = sd[0];
    for (int t = 0; t < WG; t++) {
      float acc = 0.0f;
      for (int i = t; i < seq_len; i += WG) {
        float e = expf(s[i] - gmax);
        s[i] = e;
        acc += e;
      }
      sd[t] = acc;
    }
    float total = tree_sum(sd);
    for (int i = 0; i < seq_len; i++) s[i] /= total;
  }
}

/* attnValue, src/shaders.ts:414-447 */
void vxo_attn_value(const float *scores, const float *vcache, float *out,
                    int n_heads, int n_kv_heads, int head_dim, int seq_len) {
  int rep = n_heads / n_kv_heads;
  for (int h = 0; h < n_heads; h++) {
    int kvh = h / rep;
    for (int d = 0; d < head_dim; d++) {
      float sum = 0.0f;
      for (int p = 0; p < seq_len; p++)
        sum += scores[h * seq_len + p] *
               vcache[(size_t)p * n_kv_heads * head_dim + kvh * head_dim + d];
      out[h * head_dim + d] = sum;
    }
  }
}

/* swiGLU / swiGLUOffset, src/shaders.ts:483-501, 1376-1396 */
void vxo_swiglu(float *gate, const float *up, int n) {
  for (int i = 0; i < n; i++) {
    float g = gate[i];
    float silu = g / (1.0f + expf(-g));
    gate[i] = silu * up[i];
  }
}

/* timeEmbedding, src/shaders.ts:579-602 */
void vxo_time_embedding(float *out, int dim, float t) {
  int half = dim / 2;
  const float c = (float)-9.210340371976184; /* -ln(1e4), as an f32 literal */
  for (int i = 0; i < half; i++) {
    float freq = expf(c * (float)i / (float)half);
    float angle = t * freq;
    out[i] = cosf(angle);
    out[half + i] = sinf(angle);
  }
}

/* cfgCombine, src/shaders.ts:632-648 */
void vxo_cfg_combine(float *v_cond, const float *v_uncond, int n, float alpha) {
  float beta = 1.0f - alpha;
  for (int i = 0; i < n; i++) {
    float a = alpha * v_cond[i];
    float b = beta * v_uncond[i];
    v_cond[i] = a + b;
  }
}

/* eulerStep, src/shaders.ts:611-627 */
void vxo_euler_step(float *x, const float *v, int n, float dt) {
  for (int i = 0; i < n; i++) x[i] = x[i] + v[i] * dt;
}

/* fsqQuantize, src/shaders.ts:653-673; WGSL round() is half-to-even. */
void vxo_fsq_quantize(const float *x, uint32_t *codes, int n, int levels,
                      int offset) {
  float top = (float)(levels - 1);
  for (int i = 0; i < n; i++) {
    float c = fminf(fmaxf(x[i], -1.0f), 1.0f);
    float scaled = nearbyintf((c + 1.0f) * 0.5f * top);
    float cl = fminf(fmaxf(scaled, 0.0f), top);
    codes[i] = (uint32_t)cl + (uint32_t)offset;
  }
}

/* argmax, src/shaders.ts:1154-1211: strict '>' keeps the first maximum of
 * each lane's strided run and the lower lane in the tree. */
uint32_t vxo_argmax(const float *x, int n) {
  float bv[WG];
  uint32_t bi[WG];
  for (int t = 0; t < WG; t++) {
    float best = -1e30f;
    uint32_t idx = 0;
    for (int i = t; i < n; i += WG)
      if (x[i] > best) {
        best = x[i];
        idx = (uint32_t)i;
      }
    bv[t] = best;
    bi[t] = idx;
  }
  for (int s = WG / 2; s > 0; s >>= 1)
    for (int t = 0; t < s; t++)
      if (bv[t + s] > bv[t]) {
        bv[t] = bv[t + s];
        bi[t] = bi[t + s];
      }
  return bi[0];
}

/* multiCodebookEmbed, src/shaders.ts:1878-1917 with the engine's constants
 * acoustic_base 8194, stride 23, 36 codebooks (src/engine.ts:2505-2511). */
void vxo_multi_codebook_embed(const uint16_t *table, uint32_t semantic_code,
                              const uint32_t *acoustic_codes, int dim,
                              float *out) {
  h2f_init();
  for (int i = 0; i < dim; i++) {
    float sum = 0.0f;
    sum += H(table[(size_t)semantic_code * dim + i]);
    for (int k = 0; k < 36; k++) {
      size_t row = 8194u + (size_t)k * 23u + acoustic_codes[k];
      sum += H(table[row * dim + i]);
    }
    out[i] = sum;
  }
}

/* biAttnScore / biSoftmax / biAttnValue, src/shaders.ts:684-807.
 * q [seq][n_heads*hd], k/v [seq][n_kv*hd], scores [n_heads][seq][seq],
 * out [seq][n_heads*hd]. */
void vxo_bi_attention(const float *q, const float *k, const float *v,
                      float *scores, float *out, int n_heads, int n_kv_heads,
                      int head_dim, int seq_len) {
  int rep = n_heads / n_kv_heads;
  float scale = 1.0f / sqrtf((float)head_dim);
  for (int h = 0; h < n_heads; h++)
    for (int qi = 0; qi < seq_len; qi++)
      for (int ki = 0; ki < seq_len; ki++) {
        const float *qq = q + (size_t)qi * n_heads * head_dim + h * head_dim;
        const float *kk = k + (size_t)ki * n_kv_heads * head_dim + (h / rep) * head_dim;
        float dot = 0.0f;
        for (int d = 0; d < head_dim; d++) dot += qq[d] * kk[d];
        scores[(h * seq_len + qi) * seq_len + ki] = dot * scale;
      }
  for (int h = 0; h < n_heads; h++)
    for (int qi = 0; qi < seq_len; qi++) {
      float *s = scores + (h * seq_len + qi) * seq_len;
      float m = -1e30f;
      for (int j = 0; j < seq_len; j++) m = fmaxf(m, s[j]);
      float sum = 0.0f;
      for (int j = 0; j < seq_len; j++) {
        float e = expf(s[j] - m);
        s[j] = e;
        sum += e;
      }
      for (int j = 0; j < seq_len; j++) s[j] /= sum;
    }
  for (int qi = 0; qi < seq_len; qi++)
    for (int h = 0; h < n_heads; h++)
      for (int d = 0; d < head_dim; d++) {
        const float *s = scores + (h * seq_len + qi) * seq_len;
        float sum = 0.0f;
        for (int ki = 0; ki < seq_len; ki++)
          sum += s[ki] * v[(size_t)ki * n_kv_heads * head_dim + (h / rep) * head_dim + d];
        out[(size_t)qi * n_heads * head_dim + h * head_dim + d] = sum;
      }
}

/* ======================================================================= */
/* Engine (src/engine.ts)                                                   */
/* ======================================================================= */

typedef struct {
  const uint16_t *attn_norm, *wq, *wk, *wv, *wo, *ffn_norm, *w1, *w2, *w3;
} layer_w;

typedef struct {
  char name[96];
  const uint16_t **slot;
  size_t numel;
  int is_norm;
} wslot;

struct vxo_engine {
  vxo_config c;
  int max_seq;
  int position;
  /* weights (src/engine.ts:73-103) */
  const uint16_t *tok_emb, *audio_emb, *final_norm;
  layer_w *L;
  const uint16_t *fm_input_proj, *fm_llm_proj, *fm_time_proj, *fm_norm,
      *fm_sem_out, *fm_ac_out;
  layer_w *FL;
  wslot *slots;
  int n_slots;
  uint16_t **owned; /* synthetic weights */
  int n_owned;
  /* KV cache, f32 [max_seq][kv_dim] per layer (src/engine.ts:510-530) */
  float **kv_k, **kv_v;
  /* work buffers (src/engine.ts:106-152) */
  float *hidden, *residual, *normed, *q, *k, *v, *attn_out, *scores, *gate,
      *up, *down, *logits;
  float *x_t, *velocity, *v_uncond, *time_embed, *time_proj, *x_t_proj,
      *fm_hidden, *fm_residual, *fm_normed, *fm_q, *fm_k, *fm_v, *fm_attn_out,
      *fm_scores, *fm_seq, *fm_gate, *fm_up, *fm_down, *semantic_logits;
  uint32_t semantic_argmax, argmax_result, acoustic_codes[64];
  /* batched dataflow scratch */
  float *time_proj_table; /* [nfe-1][dim] */
  int time_table_ready;
  int kv_f16; /* store K/V rows rounded to f16 (the BASELINE KV precision) */
};

void vxo_default_config(vxo_config *c) {
  c->dim = 3072;
  c->n_layers = 26;
  c->head_dim = 128;
  c->hidden_dim = 9216;
  c->n_heads = 32;
  c->n_kv_heads = 8;
  c->vocab_size = 131072;
  c->rope_theta = 1000000.0f;
  c->norm_eps = 1e-5f;
  c->fm_layers = 3;
  c->nfe = 8;
  c->cfg_alpha = 1.2f;
  c->n_acoustic_out = 36;
  c->semantic_vocab = 8320;
  c->acoustic_levels = 21;
  c->audio_vocab = 9088;
}

static void add_slot(vxo_engine *e, const char *name, const uint16_t **slot,
                     size_t numel, int is_norm) {
  wslot *s = &e->slots[e->n_slots++];
  snprintf(s->name, sizeof(s->name), "%s", name);
  s->slot = slot;
  s->numel = numel;
  s->is_norm = is_norm;
}

static void add_layer_slots(vxo_engine *e, const char *prefix, layer_w *l) {
  const vxo_config *c = &e->c;
  size_t d = (size_t)c->dim, qd = (size_t)c->n_heads * c->head_dim,
         kvd = (size_t)c->n_kv_heads * c->head_dim, hd = (size_t)c->hidden_dim;
  char nm[96];
#define SL(suffix, field, n, norm)                           \
  snprintf(nm, sizeof nm, "%s.%s", prefix, suffix);          \
  add_slot(e, nm, &l->field, n, norm);
  SL("attention_norm.weight", attn_norm, d, 1);
  SL("attention.wq.weight", wq, qd * d, 0);
  SL("attention.wk.weight", wk, kvd * d, 0);
  SL("attention.wv.weight", wv, kvd * d, 0);
  SL("attention.wo.weight", wo, d * qd, 0);
  SL("ffn_norm.weight", ffn_norm, d, 1);
  SL("feed_forward.w1.weight", w1, hd * d, 0);
  SL("feed_forward.w2.weight", w2, d * hd, 0);
  SL("feed_forward.w3.weight", w3, hd * d, 0);
#undef SL
}

static float *falloc(size_t n) {
  float *p = (float *)calloc(n ? n : 1, sizeof(float));
  if (!p) {
    fprintf(stderr, "vx_oracle: out of memory (%zu floats)\n", n);
    abort();
  }
  return p;
}

vxo_engine *vxo_create(const vxo_config *cfg, int max_seq) {
  h2f_init();
  vxo_engine *e = (vxo_engine *)calloc(1, sizeof(vxo_engine));
  e->c = *cfg;
  e->max_seq = max_seq;
  const vxo_config *c = &e->c;
  int nl = c->n_layers, fl = c->fm_layers;
  e->L = (layer_w *)calloc((size_t)nl, sizeof(layer_w));
  e->FL = (layer_w *)calloc((size_t)fl, sizeof(layer_w));
  e->slots = (wslot *)calloc((size_t)(nl + fl) * 9 + 16, sizeof(wslot));
  size_t d = (size_t)c->dim;
  add_slot(e, "mm_audio_embeddings.tok_embeddings.weight", &e->tok_emb,
           (size_t)c->vocab_size * d, 0);
  add_slot(e, "mm_audio_embeddings.audio_codebook_embeddings.embeddings.weight",
           &e->audio_emb, (size_t)c->audio_vocab * d, 0);
  add_slot(e, "norm.weight", &e->final_norm, d, 1);
  char nm[96];
  for (int i = 0; i < nl; i++) {
    snprintf(nm, sizeof nm, "layers.%d", i);
    add_layer_slots(e, nm, &e->L[i]);
  }
  add_slot(e, "acoustic_transformer.input_projection.weight", &e->fm_input_proj,
           d * (size_t)c->n_acoustic_out, 0);
  add_slot(e, "acoustic_transformer.llm_projection.weight", &e->fm_llm_proj, d * d, 0);
  add_slot(e, "acoustic_transformer.time_projection.weight", &e->fm_time_proj, d * d, 0);
  add_slot(e, "acoustic_transformer.norm.weight", &e->fm_norm, d, 1);
  add_slot(e, "acoustic_transformer.semantic_codebook_output.weight", &e->fm_sem_out,
           (size_t)c->semantic_vocab * d, 0);
  add_slot(e, "acoustic_transformer.acoustic_codebook_output.weight", &e->fm_ac_out,
           (size_t)c->n_acoustic_out * d, 0);
  for (int i = 0; i < fl; i++) {
    snprintf(nm, sizeof nm, "acoustic_transformer.layers.%d", i);
    add_layer_slots(e, nm, &e->FL[i]);
  }

  size_t kvd = (size_t)c->n_kv_heads * c->head_dim;
  size_t qd = (size_t)c->n_heads * c->head_dim;
  e->kv_k = (float **)calloc((size_t)nl, sizeof(float *));
  e->kv_v = (float **)calloc((size_t)nl, sizeof(float *));
  for (int i = 0; i < nl; i++) {
    e->kv_k[i] = falloc((size_t)max_seq * kvd);
    e->kv_v[i] = falloc((size_t)max_seq * kvd);
  }
  size_t hd = (size_t)c->hidden_dim;
  e->hidden = falloc(d);
  e->residual = falloc(d);
  e->normed = falloc(d);
  e->q = falloc(qd);
  e->k = falloc(kvd);
  e->v = falloc(kvd);
  e->attn_out = falloc(qd);
  e->scores = falloc((size_t)c->n_heads * max_seq);
  e->gate = falloc(hd);
  e->up = falloc(hd);
  e->down = falloc(d);
  e->logits = falloc((size_t)c->vocab_size);
  size_t na = (size_t)c->n_acoustic_out;
  e->x_t = falloc(na);
  e->velocity = falloc(na);
  e->v_uncond = falloc(na);
  e->time_embed = falloc(d);
  e->time_proj = falloc(d);
  e->x_t_proj = falloc(d);
  e->fm_hidden = falloc(d);
  e->fm_residual = falloc(d);
  e->fm_normed = falloc(d);
  e->fm_q = falloc(3 * qd);
  e->fm_k = falloc(3 * kvd);
  e->fm_v = falloc(3 * kvd);
  e->fm_attn_out = falloc(3 * qd);
  e->fm_scores = falloc((size_t)c->n_heads * 9);
  e->fm_seq = falloc(3 * d);
  e->fm_gate = falloc(3 * hd);
  e->fm_up = falloc(3 * hd);
  e->fm_down = falloc(3 * d);
  e->semantic_logits = falloc((size_t)c->semantic_vocab);
  e->time_proj_table = falloc((size_t)(c->nfe > 1 ? c->nfe - 1 : 1) * d);
  return e;
}

void vxo_destroy(vxo_engine *e) {
  if (!e) return;
  for (int i = 0; i < e->c.n_layers; i++) {
    free(e->kv_k[i]);
    free(e->kv_v[i]);
  }
  free(e->kv_k);
  free(e->kv_v);
  float *bufs[] = {e->hidden, e->residual, e->normed, e->q, e->k, e->v,
                   e->attn_out, e->scores, e->gate, e->up, e->down, e->logits,
                   e->x_t, e->velocity, e->v_uncond, e->time_embed,
                   e->time_proj, e->x_t_proj, e->fm_hidden, e->fm_residual,
                   e->fm_normed, e->fm_q, e->fm_k, e->fm_v, e->fm_attn_out,
                   e->fm_scores, e->fm_seq, e->fm_gate, e->fm_up, e->fm_down,
                   e->semantic_logits, e->time_proj_table};
  for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; i++) free(bufs[i]);
  for (int i = 0; i < e->n_owned; i++) free(e->owned[i]);
  free(e->owned);
  free(e->slots);
  free(e->L);
  free(e->FL);
  free(e);
}

static wslot *find_slot(const vxo_engine *e, const char *name) {
  for (int i = 0; i < e->n_slots; i++)
    if (strcmp(e->slots[i].name, name) == 0) return &e->slots[i];
  return NULL;
}

int vxo_set_weight(vxo_engine *e, const char *name, const uint16_t *data) {
  wslot *s = find_slot(e, name);
  if (!s) return -1;
  *s->slot = data;
  e->time_table_ready = 0;
  return 0;
}

size_t vxo_weight_numel(const vxo_engine *e, const char *name) {
  wslot *s = find_slot(e, name);
  return s ? s->numel : 0;
}

const uint16_t *vxo_weight(const vxo_engine *e, const char *name) {
  wslot *s = find_slot(e, name);
  return s ? *s->slot : NULL;
}

int vxo_init_synthetic(vxo_engine *e, uint64_t seed, float std) {
  e->owned = (uint16_t **)calloc((size_t)e->n_slots, sizeof(uint16_t *));
  for (int i = 0; i < e->n_slots; i++) {
    wslot *s = &e->slots[i];
    uint16_t *buf = (uint16_t *)malloc(s->numel * sizeof(uint16_t));
    if (!buf) return -1;
    vxo_gen_f16(seed, vxo_name_stream(s->name), s->numel, s->is_norm ? 1.0f : 0.0f,
                std, buf);
    e->owned[e->n_owned++] = buf;
    *s->slot = buf;
  }
  e->time_table_ready = 0;
  return 0;
}

int vxo_is_ready(const vxo_engine *e) {
  for (int i = 0; i < e->n_slots; i++)
    if (!*e->slots[i].slot) return 0;
  return 1;
}

void vxo_reset(vxo_engine *e) { e->position = 0; }
void vxo_set_kv_f16(vxo_engine *e, int on) { e->kv_f16 = on; }
int vxo_position(const vxo_engine *e) { return e->position; }
void vxo_set_position(vxo_engine *e, int pos) { e->position = pos; }
float *vxo_kv(vxo_engine *e, int layer, int which) {
  return which ? e->kv_v[layer] : e->kv_k[layer];
}
uint32_t *vxo_acoustic_codes(vxo_engine *e) { return e->acoustic_codes; }
uint32_t vxo_semantic_argmax(const vxo_engine *e) { return e->semantic_argmax; }
void vxo_set_semantic_code(vxo_engine *e, uint32_t code) { e->semantic_argmax = code; }
void vxo_set_acoustic_codes(vxo_engine *e, const uint32_t *codes) {
  memcpy(e->acoustic_codes, codes, (size_t)e->c.n_acoustic_out * sizeof(uint32_t));
}
uint32_t vxo_argmax_result(const vxo_engine *e) { return e->argmax_result; }

float *vxo_buffer(vxo_engine *e, const char *name, int *count) {
  const vxo_config *c = &e->c;
  int d = c->dim, qd = c->n_heads * c->head_dim, kvd = c->n_kv_heads * c->head_dim,
      hd = c->hidden_dim, na = c->n_acoustic_out;
  struct {
    const char *n;
    float *p;
    int cnt;
  } t[] = {
      {"hidden", e->hidden, d},
      {"residual", e->residual, d},
      {"normed", e->normed, d},
      {"q", e->q, qd},
      {"k", e->k, kvd},
      {"v", e->v, kvd},
      {"attn_out", e->attn_out, qd},
      {"scores", e->scores, c->n_heads * e->max_seq},
      {"gate", e->gate, hd},
      {"up", e->up, hd},
      {"down", e->down, d},
      {"logits", e->logits, c->vocab_size},
      {"x_t", e->x_t, na},
      {"velocity", e->velocity, na},
      {"v_uncond", e->v_uncond, na},
      {"time_embed", e->time_embed, d},
      {"time_proj", e->time_proj, d},
      {"x_t_proj", e->x_t_proj, d},
      {"fm_hidden", e->fm_hidden, d},
      {"fm_residual", e->fm_residual, d},
      {"fm_normed", e->fm_normed, d},
      {"fm_q", e->fm_q, 3 * qd},
      {"fm_k", e->fm_k, 3 * kvd},
      {"fm_v", e->fm_v, 3 * kvd},
      {"fm_attn_out", e->fm_attn_out, 3 * qd},
      {"fm_scores", e->fm_scores, c->n_heads * 9},
      {"fm_seq", e->fm_seq, 3 * d},
      {"fm_gate", e->fm_gate, 3 * hd},
      {"fm_up", e->fm_up, 3 * hd},
      {"fm_down", e->fm_down, 3 * d},
      {"semantic_logits", e->semantic_logits, c->semantic_vocab},
  };
  for (size_t i = 0; i < sizeof t / sizeof t[0]; i++)
    if (strcmp(t[i].n, name) == 0) {
      if (count) *count = t[i].cnt;
      return t[i].p;
    }
  if (count) *count = 0;
  return NULL;
}

/* backboneStep, src/engine.ts:814-1042.  Caller-visible position++ as in
 * every public caller of backboneStep (e.g. src/engine.ts:2341, 2470). */
/* One step; layer_out [n_layers][2][dim] receives the hidden state after
 * each attention and FFN residual, dbg_embed [dim] the embedding (the first
 * layer's input) and dbg_layers [n_layers][4][dim] the reference's full
 * read points attn_norm, attn_out, ffn_norm, ffn_out (each pointer may be
 * NULL). */
static void backbone_step_impl(vxo_engine *e, int token, int mode,
                               const float *precomputed, int lm_head,
                               float *layer_out, float *dbg_embed,
                               float *dbg_layers) {
  const vxo_config *c = &e->c;
  const int d = c->dim, qd = c->n_heads * c->head_dim,
            kvd = c->n_kv_heads * c->head_dim, hd = c->hidden_dim;
  const int pos = e->position;
  if (pos >= e->max_seq) {
    fprintf(stderr, "vx_oracle: position %d >= max_seq %d\n", pos, e->max_seq);
    abort();
  }
  /* embed (:832-841), optional replacement by a precomputed row (:847-854) */
  vxo_embedding(mode == 1 ? e->audio_emb : e->tok_emb, mode == 2 ? 0 : token, d,
                e->hidden);
  if (mode == 2) memcpy(e->hidden, precomputed, (size_t)d * sizeof(float));
  if (dbg_embed) memcpy(dbg_embed, e->hidden, (size_t)d * sizeof(float));
  for (int l = 0; l < c->n_layers; l++) {
    const layer_w *L = &e->L[l];
    float *dl = dbg_layers ? dbg_layers + (size_t)(4 * l) * d : NULL;
    memcpy(e->residual, e->hidden, (size_t)d * sizeof(float));
    vxo_rmsnorm(e->hidden, L->attn_norm, e->normed, d, c->norm_eps);
    if (dl) memcpy(dl, e->normed, (size_t)d * 4);
    vxo_matvec_f16(L->wq, e->normed, e->q, qd, d);
    vxo_matvec_f16(L->wk, e->normed, e->k, kvd, d);
    vxo_matvec_f16(L->wv, e->normed, e->v, kvd, d);
    vxo_rope(e->q, c->head_dim, pos, c->n_heads, c->rope_theta);
    vxo_rope(e->k, c->head_dim, pos, c->n_kv_heads, c->rope_theta);
    memcpy(e->kv_k[l] + (size_t)pos * kvd, e->k, (size_t)kvd * sizeof(float));
    memcpy(e->kv_v[l] + (size_t)pos * kvd, e->v, (size_t)kvd * sizeof(float));
    if (e->kv_f16) { /* f16 KV storage: the cached row is the f16 rounding */
      float *kr = e->kv_k[l] + (size_t)pos * kvd, *vr = e->kv_v[l] + (size_t)pos * kvd;
      for (int i = 0; i < kvd; i++) {
        kr[i] = vxo_f16_to_f32(vxo_f32_to_f16(kr[i]));
        vr[i] = vxo_f16_to_f32(vxo_f32_to_f16(vr[i]));
      }
    }
    int seq = pos + 1;
    vxo_attn_scores(e->q, e->kv_k[l], e->scores, c->n_heads, c->n_kv_heads,
                    c->head_dim, seq);
    vxo_softmax(e->scores, c->n_heads, seq);
    vxo_attn_value(e->scores, e->kv_v[l], e->attn_out, c->n_heads,
                   c->n_kv_heads, c->head_dim, seq);
    vxo_matvec_f16(L->wo, e->attn_out, e->hidden, d, qd);
    for (int i = 0; i < d; i++) e->hidden[i] = e->hidden[i] + e->residual[i];
    if (layer_out) memcpy(layer_out + (size_t)(2 * l) * d, e->hidden, (size_t)d * 4);
    if (dl) memcpy(dl + d, e->hidden, (size_t)d * 4);
    memcpy(e->residual, e->hidden, (size_t)d * sizeof(float));
    vxo_rmsnorm(e->hidden, L->ffn_norm, e->normed, d, c->norm_eps);
    if (dl) memcpy(dl + 2 * d, e->normed, (size_t)d * 4);
    vxo_matvec_f16(L->w1, e->normed, e->gate, hd, d);
    vxo_matvec_f16(L->w3, e->normed, e->up, hd, d);
    vxo_swiglu(e->gate, e->up, hd);
    vxo_matvec_f16(L->w2, e->gate, e->hidden, d, hd);
    for (int i = 0; i < d; i++) e->hidden[i] = e->hidden[i] + e->residual[i];
    if (layer_out) memcpy(layer_out + (size_t)(2 * l + 1) * d, e->hidden, (size_t)d * 4);
    if (dl) memcpy(dl + 3 * d, e->hidden, (size_t)d * 4);
  }
  vxo_rmsnorm(e->hidden, e->final_norm, e->normed, d, c->norm_eps);
  if (lm_head) {
    vxo_matvec_f16(e->tok_emb, e->normed, e->logits, c->vocab_size, d);
    e->argmax_result = vxo_argmax(e->logits, c->vocab_size);
  }
  e->position++;
}

void vxo_backbone_step_ex(vxo_engine *e, int token, int mode,
                          const float *precomputed, int lm_head,
                          float *layer_out) {
  backbone_step_impl(e, token, mode, precomputed, lm_head, layer_out, NULL, NULL);
}

/* debugBackboneLayerByLayer, src/engine.ts:2106-2287 */
void vxo_backbone_step_debug(vxo_engine *e, int token, int mode,
                             const float *precomputed, float *embed,
                             float *layers) {
  backbone_step_impl(e, token, mode, precomputed, 0, NULL, embed, layers);
}

void vxo_backbone_step(vxo_engine *e, int token, int mode,
                       const float *precomputed, int lm_head) {
  vxo_backbone_step_ex(e, token, mode, precomputed, lm_head, NULL);
}

/* Frame > 0 input of generate(), src/engine.ts:2499-2541: the 37-row
 * multi-codebook sum becomes the precomputed embedding of a step (LM head
 * skipped: generate() never reads it). */
void vxo_backbone_step_codes(vxo_engine *e) {
  float *emb = falloc((size_t)e->c.dim);
  vxo_multi_codebook_embed(e->audio_emb, e->semantic_argmax, e->acoustic_codes,
                           e->c.dim, emb);
  vxo_backbone_step(e, 0, 2, emb, 0);
  free(emb);
}

/* fmTransformerPass, src/engine.ts:1057-1225 (per-position dataflow). */
static void fm_transformer_pass(vxo_engine *e, float *velocity_out) {
  const vxo_config *c = &e->c;
  const int d = c->dim, qd = c->n_heads * c->head_dim,
            kvd = c->n_kv_heads * c->head_dim, hd = c->hidden_dim;
  const float eps = 1e-5f; /* hard-coded in the engine, :1087 */
  for (int l = 0; l < c->fm_layers; l++) {
    const layer_w *L = &e->FL[l];
    memcpy(e->fm_down, e->fm_seq, (size_t)3 * d * sizeof(float));
    for (int p = 0; p < 3; p++)
      vxo_rmsnorm(e->fm_seq + p * d, L->attn_norm, e->fm_gate + p * d, d, eps);
    for (int p = 0; p < 3; p++) {
      vxo_matvec_f16(L->wq, e->fm_gate + p * d, e->fm_q + p * qd, qd, d);
      vxo_matvec_f16(L->wk, e->fm_gate + p * d, e->fm_k + p * kvd, kvd, d);
      vxo_matvec_f16(L->wv, e->fm_gate + p * d, e->fm_v + p * kvd, kvd, d);
    }
    vxo_bi_attention(e->fm_q, e->fm_k, e->fm_v, e->fm_scores, e->fm_attn_out,
                     c->n_heads, c->n_kv_heads, c->head_dim, 3);
    for (int p = 0; p < 3; p++)
      vxo_matvec_f16(L->wo, e->fm_attn_out + p * qd, e->fm_seq + p * d, d, qd);
    for (int i = 0; i < 3 * d; i++) e->fm_seq[i] = e->fm_seq[i] + e->fm_down[i];
    memcpy(e->fm_down, e->fm_seq, (size_t)3 * d * sizeof(float));
    for (int p = 0; p < 3; p++) {
      vxo_rmsnorm(e->fm_seq + p * d, L->ffn_norm, e->fm_normed, d, eps);
      vxo_matvec_f16(L->w1, e->fm_normed, e->fm_gate + p * hd, hd, d);
      vxo_matvec_f16(L->w3, e->fm_normed, e->fm_up + p * hd, hd, d);
    }
    for (int p = 0; p < 3; p++) vxo_swiglu(e->fm_gate + p * hd, e->fm_up + p * hd, hd);
    for (int p = 0; p < 3; p++)
      vxo_matvec_f16(L->w2, e->fm_gate + p * hd, e->fm_seq + p * d, d, hd);
    for (int i = 0; i < 3 * d; i++) e->fm_seq[i] = e->fm_seq[i] + e->fm_down[i];
  }
  vxo_rmsnorm(e->fm_seq, e->fm_norm, e->fm_normed, d, eps);
  vxo_matvec_f16(e->fm_ac_out, e->fm_normed, velocity_out, c->n_acoustic_out, d);
}

/* fmForward, src/engine.ts:1240-1380, with the debugNoise path (:1266). */
void vxo_fm_forward(vxo_engine *e, const float *noise) {
  const vxo_config *c = &e->c;
  const int d = c->dim, na = c->n_acoustic_out;
  vxo_matvec_f16(e->fm_sem_out, e->normed, e->semantic_logits, c->semantic_vocab, d);
  vxo_matvec_f16(e->fm_llm_proj, e->normed, e->fm_hidden, d, d);
  memcpy(e->x_t, noise, (size_t)na * sizeof(float));
  e->semantic_argmax = vxo_argmax(e->semantic_logits, c->semantic_vocab);
  for (int step = 0; step < c->nfe - 1; step++) {
    /* JS doubles packed into an f32 uniform (:1288-1289, :437-447) */
    float t = (float)((double)step / (double)(c->nfe - 1));
    float dt = (float)(1.0 / (double)(c->nfe - 1));
    vxo_time_embedding(e->time_embed, d, t);
    vxo_matvec_f16(e->fm_time_proj, e->time_embed, e->time_proj, d, d);
    vxo_matvec_f16(e->fm_input_proj, e->x_t, e->x_t_proj, d, na);
    memcpy(e->fm_seq, e->x_t_proj, (size_t)d * 4);
    memcpy(e->fm_seq + d, e->time_proj, (size_t)d * 4);
    memcpy(e->fm_seq + 2 * d, e->fm_hidden, (size_t)d * 4);
    fm_transformer_pass(e, e->velocity);
    memcpy(e->fm_seq, e->x_t_proj, (size_t)d * 4);
    memcpy(e->fm_seq + d, e->time_proj, (size_t)d * 4);
    memset(e->fm_residual, 0, (size_t)d * 4);
    memcpy(e->fm_seq + 2 * d, e->fm_residual, (size_t)d * 4);
    fm_transformer_pass(e, e->v_uncond);
    vxo_cfg_combine(e->velocity, e->v_uncond, na, c->cfg_alpha);
    vxo_euler_step(e->x_t, e->velocity, na, dt);
  }
  vxo_fsq_quantize(e->x_t, e->acoustic_codes, na, c->acoustic_levels, 2);
}

/* ---- optimal dataflow: 6 vectors (2 CFG branches x 3 positions) per
 * weight read; identical per-element arithmetic to fm_transformer_pass. */
static void fm_pass_batched(vxo_engine *e, float *seq /* [2][3][d] */,
                            float *vel /* [2][na] */) {
  const vxo_config *c = &e->c;
  const int d = c->dim, qd = c->n_heads * c->head_dim,
            kvd = c->n_kv_heads * c->head_dim, hd = c->hidden_dim;
  const float eps = 1e-5f;
  float *res = falloc((size_t)6 * d), *nrm = falloc((size_t)6 * d);
  float *q = falloc((size_t)6 * qd), *k = falloc((size_t)6 * kvd),
        *v = falloc((size_t)6 * kvd), *ao = falloc((size_t)6 * qd);
  float *g = falloc((size_t)6 * hd), *u = falloc((size_t)6 * hd);
  float sc[32 * 9 * 2 + 64];
  const float *xs[6];
  float *ys[6];
  for (int l = 0; l < c->fm_layers; l++) {
    const layer_w *L = &e->FL[l];
    memcpy(res, seq, (size_t)6 * d * 4);
    for (int j = 0; j < 6; j++) vxo_rmsnorm(seq + j * d, L->attn_norm, nrm + j * d, d, eps);
    for (int j = 0; j < 6; j++) { xs[j] = nrm + j * d; ys[j] = q + j * qd; }
    matvec_f16_multi(L->wq, xs, ys, 6, qd, d);
    for (int j = 0; j < 6; j++) ys[j] = k + j * kvd;
    matvec_f16_multi(L->wk, xs, ys, 6, kvd, d);
    for (int j = 0; j < 6; j++) ys[j] = v + j * kvd;
    matvec_f16_multi(L->wv, xs, ys, 6, kvd, d);
    for (int b = 0; b < 2; b++)
      vxo_bi_attention(q + b * 3 * qd, k + b * 3 * kvd, v + b * 3 * kvd, sc,
                       ao + b * 3 * qd, c->n_heads, c->n_kv_heads, c->head_dim, 3);
    for (int j = 0; j < 6; j++) { xs[j] = ao + j * qd; ys[j] = seq + j * d; }
    matvec_f16_multi(L->wo, xs, ys, 6, d, qd);
    for (int i = 0; i < 6 * d; i++) seq[i] = seq[i] + res[i];
    memcpy(res, seq, (size_t)6 * d * 4);
    for (int j = 0; j < 6; j++) vxo_rmsnorm(seq + j * d, L->ffn_norm, nrm + j * d, d, eps);
    for (int j = 0; j < 6; j++) { xs[j] = nrm + j * d; ys[j] = g + j * hd; }
    matvec_f16_multi(L->w1, xs, ys, 6, hd, d);
    for (int j = 0; j < 6; j++) ys[j] = u + j * hd;
    matvec_f16_multi(L->w3, xs, ys, 6, hd, d);
    for (int j = 0; j < 6; j++) vxo_swiglu(g + j * hd, u + j * hd, hd);
    for (int j = 0; j < 6; j++) { xs[j] = g + j * hd; ys[j] = seq + j * d; }
    matvec_f16_multi(L->w2, xs, ys, 6, d, hd);
    for (int i = 0; i < 6 * d; i++) seq[i] = seq[i] + res[i];
  }
  for (int b = 0; b < 2; b++) {
    vxo_rmsnorm(seq + b * 3 * d, e->fm_norm, nrm + b * d, d, eps);
    xs[b] = nrm + b * d;
    ys[b] = vel + b * c->n_acoustic_out;
  }
  matvec_f16_multi(e->fm_ac_out, xs, ys, 2, c->n_acoustic_out, d);
  free(res); free(nrm); free(q); free(k); free(v); free(ao); free(g); free(u);
}

void vxo_fm_forward_batched(vxo_engine *e, const float *noise) {
  const vxo_config *c = &e->c;
  const int d = c->dim, na = c->n_acoustic_out;
  {
    const float *xs[1] = {e->normed};
    float *ys2[1];
    ys2[0] = e->semantic_logits;
    matvec_f16_multi(e->fm_sem_out, xs, ys2, 1, c->semantic_vocab, d);
    ys2[0] = e->fm_hidden;
    matvec_f16_multi(e->fm_llm_proj, xs, ys2, 1, d, d);
  }
  if (!e->time_table_ready) { /* input-independent: computed once */
    for (int step = 0; step < c->nfe - 1; step++) {
      float t = (float)((double)step / (double)(c->nfe - 1));
      vxo_time_embedding(e->time_embed, d, t);
      vxo_matvec_f16(e->fm_time_proj, e->time_embed, e->time_proj_table + (size_t)step * d, d, d);
    }
    e->time_table_ready = 1;
  }
  memcpy(e->x_t, noise, (size_t)na * sizeof(float));
  e->semantic_argmax = vxo_argmax(e->semantic_logits, c->semantic_vocab);
  float *seq = falloc((size_t)6 * d), *vel = falloc((size_t)2 * na);
  for (int step = 0; step < c->nfe - 1; step++) {
    float dt = (float)(1.0 / (double)(c->nfe - 1));
    vxo_matvec_f16(e->fm_input_proj, e->x_t, e->x_t_proj, d, na);
    const float *tp = e->time_proj_table + (size_t)step * d;
    for (int b = 0; b < 2; b++) {
      memcpy(seq + (b * 3 + 0) * d, e->x_t_proj, (size_t)d * 4);
      memcpy(seq + (b * 3 + 1) * d, tp, (size_t)d * 4);
      if (b == 0) memcpy(seq + 2 * d, e->fm_hidden, (size_t)d * 4);
      else memset(seq + 5 * d, 0, (size_t)d * 4);
    }
    fm_pass_batched(e, seq, vel);
    memcpy(e->velocity, vel, (size_t)na * 4);
    memcpy(e->v_uncond, vel + na, (size_t)na * 4);
    vxo_cfg_combine(e->velocity, e->v_uncond, na, c->cfg_alpha);
    vxo_euler_step(e->x_t, e->velocity, na, dt);
  }
  vxo_fsq_quantize(e->x_t, e->acoustic_codes, na, c->acoustic_levels, 2);
  free(seq);
  free(vel);
}

/* generate(), src/engine.ts:2416-2585, up to the codec decode.
 *   prefill: one backboneStep per prompt token, the voice rows replacing the
 *     embeddings of positions [audio_start, audio_start + audio_count)
 *     (:2453-2472);
 *   AUDIO kick: token 24 through the text embedding (:2478-2487);
 *   frame 0: fmForward only; frame f > 0: multi-codebook embedding of the
 *     previous frame's codes as a precomputed row, then a backboneStep
 *     (:2499-2542), then fmForward;
 *   semantic code: logits with index 0 and indices >= 8194 masked
 *     (:2556-2563), then the 256-lane tree argmax (greedy, in place of
 *     sampleTopP :2565, whose Math.random nothing can reproduce);
 *   EOS on a semantic code <= 1 (:2568-2570).
 * The FM noise of frame f is x_0[i] = vxo_gauss(noise_seed, stream("fm.noise"),
 * 36 f + i) (the debugNoise path, :1266).  Teacher forcing: with forced_sem
 * and forced_ac (n_forced frames), frame f's own codes are reported but the
 * state the next frame embeds is forced_*[f], and EOS is not taken for
 * f < n_forced.  Returns the number of frames with a non-EOS code
 * (framesGenerated); per frame f < that count (and for the EOS frame, which
 * is reported at index `return value` when max_frames allows) the optional
 * outputs receive: sem_out[f], ac_out[36 f..], x_out[36 f..] (x_t after the
 * last Euler update), normed_out[dim f..] (the backbone's final norm that
 * fed the FM), logits_out[8320 f..] (unmasked semantic logits). */
int vxo_generate(vxo_engine *e, const int32_t *tokens, int n_tokens, int audio_start,
                 int audio_count, const float *voice, int max_frames, uint64_t noise_seed,
                 int ignore_eos, const uint32_t *forced_sem, const uint32_t *forced_ac,
                 int n_forced, uint32_t *sem_out, uint32_t *ac_out, float *x_out,
                 float *normed_out, float *logits_out) {
  const vxo_config *c = &e->c;
  const int d = c->dim, na = c->n_acoustic_out, sv = c->semantic_vocab;
  const int valid = 8194; /* 8192 codebook entries + 2 specials, :2561 */
  if (n_tokens < 0 || max_frames < 0 || (long)n_tokens + max_frames + 1 > e->max_seq) return -1;
  vxo_reset(e);
  for (int i = 0; i < n_tokens; i++) {
    if (voice && audio_count > 0 && i >= audio_start && i < audio_start + audio_count)
      vxo_backbone_step(e, tokens[i], 2, voice + (size_t)(i - audio_start) * d, 0);
    else
      vxo_backbone_step(e, tokens[i], 0, NULL, 0);
  }
  vxo_backbone_step(e, 24, 0, NULL, 0);
  const uint64_t stream = vxo_name_stream("fm.noise");
  float *noise = falloc((size_t)na), *masked = falloc((size_t)sv);
  int frames = 0;
  for (int f = 0; f < max_frames; f++) {
    if (f > 0) vxo_backbone_step_codes(e);
    for (int i = 0; i < na; i++) noise[i] = vxo_gauss(noise_seed, stream, (uint64_t)f * na + i);
    vxo_fm_forward_batched(e, noise);
    memcpy(masked, e->semantic_logits, (size_t)sv * sizeof(float));
    masked[0] = -INFINITY;
    for (int i = valid; i < sv; i++) masked[i] = -INFINITY;
    const uint32_t code = vxo_argmax(masked, sv);
    if (sem_out) sem_out[f] = code;
    if (ac_out) memcpy(ac_out + (size_t)f * na, e->acoustic_codes, (size_t)na * 4);
    if (x_out) memcpy(x_out + (size_t)f * na, e->x_t, (size_t)na * 4);
    if (normed_out) memcpy(normed_out + (size_t)f * d, e->normed, (size_t)d * 4);
    if (logits_out) memcpy(logits_out + (size_t)f * sv, e->semantic_logits, (size_t)sv * 4);
    const int forced = forced_sem && forced_ac && f < n_forced;
    if (code <= 1 && !ignore_eos && !forced) break;
    frames++;
    /* the state the next frame embeds (:2573-2575; acoustic codes stay in
     * W.acoustic_codes from fmForward) */
    if (forced) {
      e->semantic_argmax = forced_sem[f];
      memcpy(e->acoustic_codes, forced_ac + (size_t)f * na, (size_t)na * 4);
    } else {
      e->semantic_argmax = code;
    }
  }
  free(noise);
  free(masked);
  return frames;
}
