// vx_codec.h -- the codec decoder (semantic + acoustic codes -> 24 kHz
// waveform) on MFMA: codecDecode, src/engine.ts:1402-1713, with the codec
// shaders of src/shaders.ts:817-1110, 1432-1868.
//
// Every projection and convolution is one f16 x f16 -> f32 GEMM on the
// matrix cores, the hand-written kernels of vx_gemm.h shared with the
// prefill: the f16 weights times the activations in hi/lo f16 form, so
// products keep f32 accuracy. A GEMM may leave its sum in up to 8 K-slice
// partials; the epilogue kernels below (template parameter NS) add them in
// slice order, so every result is bit-reproducible.
//   - the causal convs become GEMMs over an im2col B (k-major: column t holds
//     x[t - (k_size-1) + kk][ci] at k = kk * c_in + ci) with the weights
//     reordered to match once after loading; their weight norm g/||w|| is
//     one scale per output row, applied in the epilogue;
//   - the stride-2 transposed conv (kernel 4) gives output step 2 tau + r
//     from input steps tau (tap r) and tau - 1 (tap r + 2): one GEMM of
//     2048 rows (both parities) over B = [x[tau]; x[tau - 1]] scaled by the
//     per-input-channel weight norm;
//   - the input conv's B is gathered straight from the codes (vqLookup,
//     fsqDequant and concatCodecInput fused into the packing).
// Tokens are processed in column chunks of at most CX_MAXT; a chunk's B
// holds nc = 2 * nt columns (nt = tokens rounded up to 128, hi then lo),
// each column's K halves contiguous; the GEMM output C is [nc][M].
#pragma once
#include "vx_prefill.h"

namespace vx {

// codec dimensions (src/types.ts:98-122)
constexpr int CD = 1024, CHID = 4096, CNH = 8, CHDIM = 128;
constexpr int CSEM = 8192, CSEMD = 256, CIN = CSEMD + NAC;  // 292 input channels
constexpr int CPATCH = 240, CPATCH_ROWS = 256;  // output conv rows, padded to the GEMM tile
constexpr int CK_IN = 3, CK_OUT = 7, CK_UP = 4;
constexpr int CKIN = 896;            // CIN * CK_IN = 876, rounded up to 32
constexpr int CKOUT = CD * CK_OUT;   // 7168
constexpr int CKUP = 2 * CD;         // input steps tau and tau - 1
constexpr int CX_STAGES = 4, CX_LPS = 2;
constexpr int CX_FRAME_SAMPLES = 8 * CPATCH;  // 1920 samples = 80 ms at 24 kHz
constexpr int CX_MAXT = 1024;                 // tokens per GEMM chunk
constexpr int CX_NC = 2 * CX_MAXT;
constexpr size_t CX_CCAP = (size_t)CX_NC * 2 * CHID;  // GEMM output floats
constexpr float CX_NORM_EPS = 0.01f, CX_QK_EPS = 1e-6f;
static_assert(CKIN % 32 == 0 && CKIN >= CIN * CK_IN, "input conv k padding");

// output (token t, row m) of a chunk's GEMM: the sum of its NS K-slice
// blocks [nc / 2][ldc] (vx_gemm.h), in order
template <int NS>
__device__ __forceinline__ float cx_val(const float *C, int ldc, int nc, int t, int m) {
  float v[NS];
#pragma unroll
  for (int s = 0; s < NS; s++) v[s] = C[((size_t)s * (nc >> 1) + t) * ldc + m];
  float y = v[0];
#pragma unroll
  for (int s = 1; s < NS; s++) y += v[s];
  return y;
}

// outputs m .. m + 7 (m % 8 == 0) of token t, the same in-order sums as
// cx_val, from two 16-byte loads per K-slice block
template <int NS>
__device__ __forceinline__ void cx_val8(const float *C, int ldc, int nc, int t, int m, float (&y)[8]) {
  f32x4 a[NS], b[NS];
#pragma unroll
  for (int s = 0; s < NS; s++) {
    const float *p = C + ((size_t)s * (nc >> 1) + t) * ldc + m;
    a[s] = *(const f32x4 *)p;
    b[s] = *(const f32x4 *)(p + 4);
  }
#pragma unroll
  for (int e = 0; e < 4; e++) {
    y[e] = a[0][e];
    y[4 + e] = b[0][e];
  }
#pragma unroll
  for (int s = 1; s < NS; s++)
#pragma unroll
    for (int e = 0; e < 4; e++) {
      y[e] += a[s][e];
      y[4 + e] += b[s][e];
    }
}

// 8 consecutive f32 / f16 values from 16-byte aligned addresses
__device__ __forceinline__ void cx_load8(const float *x, float (&y)[8]) {
  const f32x4 a = *(const f32x4 *)x, b = *(const f32x4 *)(x + 4);
#pragma unroll
  for (int e = 0; e < 4; e++) {
    y[e] = a[e];
    y[4 + e] = b[e];
  }
}
__device__ __forceinline__ void cx_load8h(const uint16_t *g, float (&y)[8]) {
  const h8 w = *(const h8 *)g;
#pragma unroll
  for (int e = 0; e < 8; e++) y[e] = (float)w[e];
}

// k group kb (8 halves) of columns t (hi) and nt + t (lo); kg = K / 8
__device__ __forceinline__ void cx_put(h8 *B, int nc, int kg, int kb, int t, const float (&y)[8]) {
  h8 hi, lo;
  split_n<8>(y, hi, lo);
  B[(size_t)t * kg + kb] = hi;
  B[(size_t)((nc >> 1) + t) * kg + kb] = lo;
}

// ------------------------------------------------------------- packing
// B from rows t0 + t of X [*][K], optionally RMS-normalised with gains g
// (batchedRmsNorm, src/shaders.ts:1646-1692).  Grid: nt blocks of 256.
template <bool NORM>
__global__ __launch_bounds__(256) void cx_pack_kernel(const float *X, int K, int t0, int n, int nc,
                                                      const uint16_t *g, float eps, h8 *B) {
  const int t = blockIdx.x, tid = threadIdx.x;
  const bool live = t < n;
  const float *x = X + (size_t)(t0 + t) * K;
  float r = 1.0f;
  if (NORM && live) {
    __shared__ float red[4];
    float s = 0.f;
    for (int k = tid; k < K; k += 256) s = fmaf(x[k], x[k], s);
    s = wave_sum(s);
    if ((tid & 63) == 0) red[tid >> 6] = s;
    __syncthreads();
    r = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)K + eps);
  }
  for (int kb = tid; kb < K / 8; kb += 256) {
    float y[8];
    if (live) {
      cx_load8(x + kb * 8, y);
      if (NORM) {
        float gv[8];
        cx_load8h(g + kb * 8, gv);
#pragma unroll
        for (int e = 0; e < 8; e++) y[e] = y[e] * r * gv[e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; e++) y[e] = 0.f;
    }
    cx_put(B, nc, K / 8, kb, t, y);
  }
}

// input channel ci of frame tau: the normalised semantic codebook row of its
// semantic code (vqLookup, src/shaders.ts:817-845; rows past the 8192-entry
// table read as zero), then the 36 dequantised acoustic values
// (fsqDequant, src/shaders.ts:891-914: u32 code - 2, * 2 / (levels - 1) - 1)
__device__ __forceinline__ float cx_feature(const uint16_t *cbn, const uint32_t *sem,
                                            const uint32_t *ac, int levels, int tau, int ci) {
  if (ci < CSEMD) {
    const uint32_t c = sem[tau];
    return c < (uint32_t)CSEM ? h2f(cbn[(size_t)c * CSEMD + ci]) : 0.f;
  }
  const uint32_t c = ac[(size_t)tau * NAC + (ci - CSEMD)] - 2u;
  return (float)c * 2.0f / (float)(levels - 1) - 1.0f;
}

// im2col B of the input conv (k = 3) straight from the codes.
// Grid: nt blocks of 128.
__global__ __launch_bounds__(128) void cx_pack_in_kernel(const uint16_t *cbn, const uint32_t *sem,
                                                         const uint32_t *ac, int levels, int t0,
                                                         int n, int nc, h8 *B) {
  const int t = blockIdx.x, tau = t0 + t;
  for (int kb = threadIdx.x; kb < CKIN / 8; kb += blockDim.x) {
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const int k = kb * 8 + e, kk = k / CIN, ci = k - kk * CIN;
      const int src = tau - (CK_IN - 1) + kk;
      y[e] = (t < n && k < CIN * CK_IN && src >= 0) ? cx_feature(cbn, sem, ac, levels, src, ci) : 0.f;
    }
    cx_put(B, nc, CKIN / 8, kb, t, y);
  }
}

// B of the transposed conv: k = j * CD + ci holds scale[ci] * x[tau - j][ci].
// Grid: nt blocks of 256.
__global__ __launch_bounds__(256) void cx_pack_up_kernel(const float *X, const float *scale, int t0,
                                                         int n, int nc, h8 *B) {
  const int t = blockIdx.x, tau = t0 + t;
  for (int kb = threadIdx.x; kb < CKUP / 8; kb += 256) {
    const int j = kb / (CD / 8), ci0 = (kb - j * (CD / 8)) * 8, src = tau - j;
    const bool ok = t < n && src >= 0;
    float y[8];
    if (ok) {
      float sc[8];
      cx_load8(X + (size_t)src * CD + ci0, y);
      cx_load8(scale + ci0, sc);
#pragma unroll
      for (int e = 0; e < 8; e++) y[e] = sc[e] * y[e];
    } else {
#pragma unroll
      for (int e = 0; e < 8; e++) y[e] = 0.f;
    }
    cx_put(B, nc, CKUP / 8, kb, t, y);
  }
}

// im2col B of the output conv (k = 7): k = kk * CD + ci holds
// x[tau - 6 + kk][ci].  Grid: nt blocks of 256.
__global__ __launch_bounds__(256) void cx_pack_out_kernel(const float *X, int t0, int n, int nc,
                                                          h8 *B) {
  const int t = blockIdx.x, tau = t0 + t;
  for (int kb = threadIdx.x; kb < CKOUT / 8; kb += 256) {
    const int kk = kb / (CD / 8), ci0 = (kb - kk * (CD / 8)) * 8, src = tau - (CK_OUT - 1) + kk;
    float y[8];
    if (t < n && src >= 0) {
      cx_load8(X + (size_t)src * CD + ci0, y);
    } else {
#pragma unroll
      for (int e = 0; e < 8; e++) y[e] = 0.f;
    }
    cx_put(B, nc, CKOUT / 8, kb, t, y);
  }
}

// ----------------------------------------------------------- epilogues
// out[(t0 + t) * ldo + m] = rs[m] * y (conv weight norm g / ||w|| per
// output channel), m < mv.  Grid: (n, ceil(mv / 256)).
template <int NS>
__global__ void cx_scale_rows_epi_kernel(const float *C, int ldc, int nc, int t0, const float *rs,
                                         int mv, float *out, int ldo) {
  const int t = blockIdx.x, m = blockIdx.y * blockDim.x + threadIdx.x;
  if (m < mv) out[(size_t)(t0 + t) * ldo + m] = rs[m] * cx_val<NS>(C, ldc, nc, t, m);
}

// transposed conv output: step 2 (t0 + t) + r, channel co from row r * CD + co.
// Grid: (n, 2 * CD / 256).
template <int NS>
__global__ void cx_up_epi_kernel(const float *C, int nc, int t0, float *out) {
  const int t = blockIdx.x, m = blockIdx.y * blockDim.x + threadIdx.x;
  const int r = m / CD, co = m - r * CD;
  out[(size_t)(2 * (t0 + t) + r) * CD + co] = cx_val<NS>(C, 2 * CD, nc, t, m);
}

// layer scale + residual (batchedLayerScale, src/shaders.ts:1755-1781):
// X = y * scale + X.  Grid: (n, CD / 256).
template <int NS>
__global__ void cx_resid_epi_kernel(const float *C, int nc, int t0, const uint16_t *scale,
                                    float *X) {
  const int t = blockIdx.x, m = blockIdx.y * blockDim.x + threadIdx.x;
  float *x = X + (size_t)(t0 + t) * CD + m;
  *x = cx_val<NS>(C, CD, nc, t, m) * h2f(scale[m]) + *x;
}

// q, k, v from the stacked projection, q and k RMS-normalised per head
// (qkNorm, src/shaders.ts:1787-1830: weight [CNH * CHDIM] read at h * CHDIM).
// One wave per (token, part, head); grid (n, 3 * CNH / 4) of 256.
template <int NS>
__global__ __launch_bounds__(256) void cx_qkv_epi_kernel(const float *C, int nc, int t0,
                                                         const uint16_t *qn, const uint16_t *kn,
                                                         float *Q, float *K, float *V) {
  const int t = blockIdx.x, gi = blockIdx.y * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int part = gi / CNH, h = gi - part * CNH, d = 2 * lane;
  const int m = part * CD + h * CHDIM + d;
  float y0 = cx_val<NS>(C, 3 * CD, nc, t, m), y1 = cx_val<NS>(C, 3 * CD, nc, t, m + 1);
  if (part < 2) {
    const float ss = wave_sum(y0 * y0 + y1 * y1);
    const float r = 1.0f / sqrtf(ss / (float)CHDIM + CX_QK_EPS);
    const uint16_t *w = (part == 0 ? qn : kn) + h * CHDIM + d;
    y0 = y0 * r * h2f(w[0]);
    y1 = y1 * r * h2f(w[1]);
  }
  float *dst = part == 0 ? Q : part == 1 ? K : V;
  *(float2 *)(dst + (size_t)(t0 + t) * CD + h * CHDIM + d) = make_float2(y0, y1);
}

// SwiGLU of the stacked gate/up projection (batchedSwiGLU,
// src/shaders.ts:1697-1716), written as the packed B of the down projection
// (k = hidden unit).  Grid: (nt, CHID / 8 / 256) of 256; columns t >= n are 0.
template <int NS>
__global__ __launch_bounds__(256) void cx_swiglu_epi_kernel(const float *C, int nc, int n, h8 *B) {
  const int t = blockIdx.x, kb = blockIdx.y * 256 + threadIdx.x;
  float y[8];
  if (t < n) {
    float g[8], u[8];
    cx_val8<NS>(C, 2 * CHID, nc, t, kb * 8, g);
    cx_val8<NS>(C, 2 * CHID, nc, t, CHID + kb * 8, u);
#pragma unroll
    for (int e = 0; e < 8; e++) y[e] = g[e] / (1.0f + expf(-g[e])) * u[e];
  } else {
#pragma unroll
    for (int e = 0; e < 8; e++) y[e] = 0.f;
  }
  cx_put(B, nc, CHID / 8, kb, t, y);
}

// ----------------------------------------------------------- attention
// Windowed causal attention with ALiBi biases (alibiAttnScore, codecSoftmax,
// codecAttnValue, src/shaders.ts:1432-1585): keys ki in
// [max(0, qi - W + 1), qi], score q.k / sqrt(128) - 2^(-8(h+1)/8) (qi - ki).
// One wave per (query, head), lane l holding dims 2l, 2l + 1.
// Grid: (T, CNH / 4) of 256; W <= 16.
constexpr int CX_MAXW = 16;
__global__ __launch_bounds__(256) void cx_attn_kernel(const float *Q, const float *K,
                                                      const float *V, int W, float *O) {
  const int qi = blockIdx.x, h = blockIdx.y * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  const size_t off = (size_t)h * CHDIM + 2 * lane;
  const float2 q = *(const float2 *)(Q + (size_t)qi * CD + off);
  const int k0 = qi + 1 > W ? qi - W + 1 : 0;
  const float scale = 1.0f / sqrtf((float)CHDIM);
  const float slope = exp2f(-8.0f * (float)(h + 1) / (float)CNH);
  float s[CX_MAXW];
  float mx = -1e30f;
#pragma unroll
  for (int j = 0; j < CX_MAXW; j++) {
    float sc = -1e30f;
    const int ki = k0 + j;
    if (j < W && ki <= qi) {
      const float2 k = *(const float2 *)(K + (size_t)ki * CD + off);
      const float dot = wave_sum(q.x * k.x + q.y * k.y);
      sc = dot * scale + (-slope * (float)(qi - ki));
    }
    s[j] = sc;
    if (j < W) mx = fmaxf(mx, sc);
  }
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < CX_MAXW; j++) {
    s[j] = j < W ? expf(s[j] - mx) : 0.f;
    sum += s[j];
  }
  float2 o = make_float2(0.f, 0.f);
#pragma unroll
  for (int j = 0; j < CX_MAXW; j++) {
    const int ki = k0 + j;
    if (j < W && ki <= qi) {
      const float p = s[j] / sum;
      const float2 v = *(const float2 *)(V + (size_t)ki * CD + off);
      o.x += p * v.x;
      o.y += p * v.y;
    }
  }
  *(float2 *)(O + (size_t)qi * CD + off) = o;
}

// the concatenated input features [T][292] (debugCodecDecode's "concat")
__global__ void cx_concat_kernel(const uint16_t *cbn, const uint32_t *sem, const uint32_t *ac,
                                 int levels, int T, float *out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < T * CIN) out[i] = cx_feature(cbn, sem, ac, levels, i / CIN, i % CIN);
}

// ------------------------------------------------ weight preparation
// normalizeCodebook (src/shaders.ts:851-885): f16(sum / max(usage, 1e-5))
__global__ void cx_vq_norm_kernel(const uint16_t *sum, const uint16_t *usage, uint16_t *out) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < (size_t)CSEM * CSEMD;
       i += (size_t)gridDim.x * blockDim.x) {
    const float u = fmaxf(h2f(usage[i / CSEMD]), 1e-5f);
    const _Float16 r = (_Float16)(h2f(sum[i]) / u);
    out[i] = __builtin_bit_cast(uint16_t, r);
  }
}

// causal conv weight norm per output row (causalConv1d, src/shaders.ts:
// 941-957): rs = g / sqrt(sum over pairs of (a^2 + b^2) + 1e-12), rows >= mv
// zero.  One thread per row.
__global__ void cx_conv_rowscale_kernel(const uint16_t *w, const uint16_t *g, int mv, int K,
                                        int rows, float *rs) {
  const int co = blockIdx.x * blockDim.x + threadIdx.x;
  if (co >= rows) return;
  if (co >= mv) {
    rs[co] = 0.f;
    return;
  }
  const uint16_t *wr = w + (size_t)co * K;
  float ss = 0.f;
  for (int p = 0; p < K / 2; p++) {
    const float a = h2f(wr[2 * p]), b = h2f(wr[2 * p + 1]);
    ss += a * a + b * b;
  }
  rs[co] = (1.0f / sqrtf(ss + 1e-12f)) * h2f(g[co]);
}

// transposed conv weight norm per input channel (convTransposeNormScale,
// src/shaders.ts:1009-1058, same 256-lane strided sums and tree):
// scale[ci] = g[ci] / ||w[ci, :, :]||.  One block of 256 per channel.
__global__ __launch_bounds__(256) void cx_up_scale_kernel(const uint16_t *w, const uint16_t *g,
                                                          float *scale) {
  __shared__ float sd[256];
  const int ci = blockIdx.x, tid = threadIdx.x, n = CD * CK_UP;
  const uint16_t *wr = w + (size_t)ci * n;
  float ss = 0.f;
  for (int i = tid; i < n; i += 256) {
    const float v = h2f(wr[i]);
    ss += v * v;
  }
  sd[tid] = ss;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (tid < s) sd[tid] += sd[tid + s];
    __syncthreads();
  }
  if (tid == 0) scale[ci] = h2f(g[ci]) * (1.0f / sqrtf(sd[0] + 1e-12f));
}

// A of the input conv: [CD][CKIN], A[co][kk * CIN + ci] = w[co][ci][kk]
__global__ void cx_reorder_in_kernel(const uint16_t *w, uint16_t *A) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < (size_t)CD * CKIN;
       i += (size_t)gridDim.x * blockDim.x) {
    const int co = (int)(i / CKIN), k = (int)(i % CKIN);
    uint16_t v = 0;
    if (k < CIN * CK_IN) {
      const int kk = k / CIN, ci = k - kk * CIN;
      v = w[((size_t)co * CIN + ci) * CK_IN + kk];
    }
    A[i] = v;
  }
}

// A of the output conv: [CPATCH_ROWS][CKOUT], A[co][kk * CD + ci] =
// w[co][ci][kk], rows >= CPATCH zero
__global__ void cx_reorder_out_kernel(const uint16_t *w, uint16_t *A) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < (size_t)CPATCH_ROWS * CKOUT;
       i += (size_t)gridDim.x * blockDim.x) {
    const int co = (int)(i / CKOUT), k = (int)(i % CKOUT);
    const int kk = k / CD, ci = k - kk * CD;
    A[i] = co < CPATCH ? w[((size_t)co * CD + ci) * CK_OUT + kk] : (uint16_t)0;
  }
}

// A of a transposed conv: [2 * CD][CKUP], A[r * CD + co][j * CD + ci] =
// w[ci][co][r + 2 j] (w is [c_in][c_out][4])
__global__ void cx_reorder_up_kernel(const uint16_t *w, uint16_t *A) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < (size_t)2 * CD * CKUP;
       i += (size_t)gridDim.x * blockDim.x) {
    const int row = (int)(i / CKUP), k = (int)(i % CKUP);
    const int r = row / CD, co = row - r * CD, j = k / CD, ci = k - j * CD;
    A[i] = w[((size_t)ci * CD + co) * CK_UP + r + 2 * j];
  }
}

}  // namespace vx
