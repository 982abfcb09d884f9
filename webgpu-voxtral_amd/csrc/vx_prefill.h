// vx_prefill.h -- batched prefill of the backbone on MFMA.  The reference
// prefills one token per backboneStep (src/engine.ts:2457-2472); here a
// chunk of up to PF_MAXT prompt tokens goes through each layer at once, so
// every weight is read once per chunk and the projections are GEMMs:
//   C[col][m] = sum_k W[m][k] * B[k][col]
// on v_mfma_f32_16x16x32_f16.  W is the layer's f16 weight matrix
// (row-major, as loaded); B holds the chunk's activations in the packed
// hi/lo form of the FM GEMMs (column t = f16(y_t), column PF_MAXT + t =
// f16(y_t - hi)), so the product keeps f32 accuracy.  Small per-token
// kernels do RMSNorm + packing, RoPE + K/V writes, residual adds, SwiGLU and
// the causal attention.  The result (K/V cache rows, residual stream, final
// norm of the last token, position) equals that of the per-token steps up to
// f32 summation order.
#pragma once
#include "vx_kernels.h"

namespace vx {

constexpr int PF_MAXT = 256;           // tokens per chunk
constexpr int PF_NC = 2 * PF_MAXT;     // B columns (hi, lo)
constexpr int PF_BM = 128, PF_BN = 256;  // block tile: rows x columns
static_assert(PF_NC % PF_BN == 0, "column tiles");

// ------------------------------------------------------------ the GEMM
// Block: 4 waves in 2 x 2, wave tile 64 rows x 128 columns (4 x 8 tiles of
// 16 x 16); k in chunks of 32 staged through LDS as [k group][row|col][8],
// double-buffered, with the global loads two chunks ahead.  The k range is
// split S ways over blockIdx.z (S = gridDim.z) so that narrow matrices fill
// the chip; slab s of C holds the partial sum of split s.  B has nc columns
// (a multiple of PF_BN; the prefill uses PF_NC).
// Grid: (M / PF_BM, nc / PF_BN, S).  C: [S][nc][ldc] f32.
template <int K>
__global__ __launch_bounds__(256) void pf_gemm_kernel(const uint16_t *W, const h8 *B, float *C,
                                                      int ldc, int nc) {
  static_assert(K % 32 == 0, "k chunks");
  const int S = gridDim.z, NCH = K / 32 / S, ch0 = blockIdx.z * NCH;
  C += (size_t)blockIdx.z * nc * ldc;
  __shared__ __attribute__((aligned(16))) h8 As[2][4][PF_BM];
  __shared__ __attribute__((aligned(16))) h8 Bs[2][4][PF_BN];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = wave >> 1, wc = wave & 1;
  const int m0 = blockIdx.x * PF_BM, n0 = blockIdx.y * PF_BN;
  const int r16 = lane & 15, g = lane >> 4;

  // global -> register staging of one k chunk (2 A pieces, 4 B pieces per
  // thread) into register set r
  u32x4 ra[2][2], rb[2][4];
  auto gload = [&](int ch, int r) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int p = tid + 256 * i, row = p >> 2, kg = p & 3;
      ra[r][i] = *(const u32x4 *)(W + (size_t)(m0 + row) * K + (ch0 + ch) * 32 + kg * 8);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int p = tid + 256 * i, kg = p >> 8, col = p & 255;
      rb[r][i] = *(const u32x4 *)(B + (size_t)((ch0 + ch) * 4 + kg) * nc + n0 + col);
    }
  };
  auto lstore = [&](int buf, int r) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int p = tid + 256 * i;
      As[buf][p & 3][p >> 2] = __builtin_bit_cast(h8, ra[r][i]);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int p = tid + 256 * i;
      Bs[buf][p >> 8][p & 255] = __builtin_bit_cast(h8, rb[r][i]);
    }
  };

  f32x4 acc[4][8];
#pragma unroll
  for (int t = 0; t < 4; t++)
#pragma unroll
    for (int c = 0; c < 8; c++) acc[t][c] = f32x4{0.f, 0.f, 0.f, 0.f};

  // chunk ch is in LDS buffer ch & 1 when iteration ch starts; chunk ch + 1
  // in register set (ch + 1) & 1; chunk ch + 2 is loaded into set ch & 1
  gload(0, 0);
  if (NCH > 1) gload(1, 1);
  lstore(0, 0);
  __syncthreads();
  for (int ch = 0; ch < NCH; ch++) {
    const int buf = ch & 1;
    if (ch + 2 < NCH) {
      if (buf) gload(ch + 2, 1);
      else gload(ch + 2, 0);
    }
    h8 af[4];
#pragma unroll
    for (int t = 0; t < 4; t++) af[t] = As[buf][g][wr * 64 + t * 16 + r16];
#pragma unroll
    for (int c = 0; c < 8; c++) {
      const h8 bf = Bs[buf][g][wc * 128 + c * 16 + r16];
#pragma unroll
      for (int t = 0; t < 4; t++)
        acc[t][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[t], bf, acc[t][c], 0, 0, 0);
    }
    if (ch + 1 < NCH) {
      if (buf) lstore(0, 0);
      else lstore(1, 1);
    }
    __syncthreads();
  }
  // D tile (t, c): lane holds rows 4*(lane/16)+j of column lane%16
#pragma unroll
  for (int t = 0; t < 4; t++)
#pragma unroll
    for (int c = 0; c < 8; c++) {
      const int col = n0 + wc * 128 + c * 16 + r16, row = m0 + wr * 64 + t * 16 + 4 * g;
      *(f32x4 *)(C + (size_t)col * ldc + row) = acc[t][c];
    }
}

// value of output (token t, row m): hi and lo columns of the S split slabs,
// summed in a fixed order
__device__ __forceinline__ float pf_c(const float *C, int ldc, int S, int t, int m) {
  float y = 0.f;
  for (int s = 0; s < S; s++, C += (size_t)PF_NC * ldc)
    y += C[(size_t)t * ldc + m] + C[(size_t)(PF_MAXT + t) * ldc + m];
  return y;
}

// ------------------------------------------------------- per-token kernels
// X[t] = token embedding row, or voice row v = t + tok0 - vstart for the
// tokens inside [vstart, vstart + vcount) (src/engine.ts:2457-2472)
__global__ void pf_embed_kernel(const uint16_t *table, const int32_t *tokens, const float *voice,
                                int vstart, int vcount, int tok0, float *X) {
  const int t = blockIdx.x, i = blockIdx.y * blockDim.x + threadIdx.x;
  const int gi = tok0 + t;
  float v;
  if (voice && gi >= vstart && gi < vstart + vcount)
    v = voice[(size_t)(gi - vstart) * DIM + i];
  else
    v = h2f(table[(size_t)tokens[t] * DIM + i]);
  X[(size_t)t * DIM + i] = v;
}

// B columns t and PF_MAXT + t from row t of X (K values), optionally
// RMS-normalised with gains g (rmsNorm, src/shaders.ts:137-183); columns of
// tokens t >= n are zero.  Grid: PF_MAXT blocks of 256.
template <bool NORM>
__global__ __launch_bounds__(256) void pf_pack_kernel(const float *X, int K, int n,
                                                      const uint16_t *g, float eps, h8 *B) {
  const int t = blockIdx.x, tid = threadIdx.x;
  const float *x = X + (size_t)t * K;
  float r = 1.0f;
  if (NORM && t < n) {
    __shared__ float red[4];
    float s = 0.f;
    for (int k = tid; k < K; k += 256) s = fmaf(x[k], x[k], s);
    s = wave_sum(s);
    if ((tid & 63) == 0) red[tid >> 6] = s;
    __syncthreads();
    r = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)K + eps);
  }
  for (int kb = tid; kb < K / 8; kb += 256) {
    h8 hi, lo;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const int k = kb * 8 + e;
      const float y = t < n ? (NORM ? x[k] * r * h2f(g[k]) : x[k]) : 0.f;
      hi[e] = (_Float16)y;
      lo[e] = (_Float16)(y - (float)hi[e]);
    }
    B[(size_t)kb * PF_NC + t] = hi;
    B[(size_t)kb * PF_NC + PF_MAXT + t] = lo;
  }
}

// QKV outputs: interleaved rope of q and k at position pos0 + t
// (src/shaders.ts:224-256), q -> Q[t][QD], k and v -> cache rows pos0 + t.
// Grid: (n, QKV_ROWS / 2 / 256), one row pair per thread.
__global__ void pf_qkv_epi_kernel(const float *C, int S, float *Q, void *kc, void *vc, int kv_f32,
                                  int max_seq, int pos0, const float *inv_freq) {
  const int t = blockIdx.x, row = 2 * (blockIdx.y * blockDim.x + threadIdx.x);
  const float y0 = pf_c(C, QKV_ROWS, S, t, row), y1 = pf_c(C, QKV_ROWS, S, t, row + 1);
  const int pos = pos0 + t;
  if (row < QD + KVD) {
    const float ang = (float)pos * inv_freq[(row & (HD - 1)) >> 1];
    const float cs = cosf(ang), sn = sinf(ang);
    const float r0 = y0 * cs - y1 * sn, r1 = y0 * sn + y1 * cs;
    if (row < QD) {
      Q[(size_t)t * QD + row] = r0;
      Q[(size_t)t * QD + row + 1] = r1;
    } else {
      kv_store2(kc, kv_f32, max_seq, row - QD, pos, r0, r1);
    }
  } else {
    kv_store2(vc, kv_f32, max_seq, row - QD - KVD, pos, y0, y1);
  }
}

// X[t][m] += output (m < M).  Grid: (n, M / 256).
__global__ void pf_resid_epi_kernel(const float *C, int M, int S, float *X) {
  const int t = blockIdx.x, m = blockIdx.y * blockDim.x + threadIdx.x;
  X[(size_t)t * M + m] += pf_c(C, M, S, t, m);
}

// act[t][m] = silu(gate) * up for the stacked [W1; W3] output (ldc = 2 HID).
// Grid: (n, HID / 256).
__global__ void pf_swiglu_epi_kernel(const float *C, float *act) {
  const int t = blockIdx.x, m = blockIdx.y * blockDim.x + threadIdx.x;
  const float gt = pf_c(C, 2 * HID, 1, t, m), up = pf_c(C, 2 * HID, 1, t, HID + m);
  act[(size_t)t * HID + m] = (gt / (1.0f + expf(-gt))) * up;
}

// Causal attention of the chunk: query t (position pos0 + t) over keys
// 0..pos0 + t of the cache.  Grid (n, NKV), 4 waves = the 4 query heads of
// the KV head; keys in LDS tiles of AT_T with an online softmax.
template <typename KVT>
__global__ __launch_bounds__(256) void pf_attn_kernel(const float *Q, const void *kc, const void *vc,
                                                      int max_seq, int pos0, float *out) {
  using G = KvTile<KVT>;
  const int t = blockIdx.x, kvh = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int h = kvh * (NH / NKV) + wave;
  const int p1 = pos0 + t + 1;
  __shared__ __attribute__((aligned(16))) float qs[4][HD];
  __shared__ __attribute__((aligned(16))) KVT ks[AT_T * G::LDW];
  __shared__ __attribute__((aligned(16))) KVT vs[AT_T * G::LDW];
  __shared__ float ps[4][AT_T];
  const float scale = 1.0f / sqrtf((float)HD);
  const KVT *Kb = (const KVT *)kc + (size_t)kvh * max_seq * HD;
  const KVT *Vb = (const KVT *)vc + (size_t)kvh * max_seq * HD;
  u32x4 kr[G::CPT], vr[G::CPT];
  attn_load_tile<KVT>(Kb, Vb, 0, min(AT_T, p1), tid, kr, vr);
  qs[wave][lane * 2] = Q[(size_t)t * QD + h * HD + lane * 2];
  qs[wave][lane * 2 + 1] = Q[(size_t)t * QD + h * HD + lane * 2 + 1];
  const int key = lane & (AT_T - 1), half = lane >> 5;
  float m = -INFINITY, l = 0.f, o0 = 0.f, o1 = 0.f;
  for (int pb = 0; pb < p1; pb += AT_T) {
    const int n = min(AT_T, p1 - pb);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < G::CPT; i++) {
      const int id = tid + 256 * i, row = id / G::CPR, col = id % G::CPR;
      *(u32x4 *)(ks + row * G::LDW + col * G::EPC) = kr[i];
      *(u32x4 *)(vs + row * G::LDW + col * G::EPC) = vr[i];
    }
    if (pb + AT_T < p1) attn_load_tile<KVT>(Kb, Vb, pb + AT_T, min(AT_T, p1 - pb - AT_T), tid, kr, vr);
    __syncthreads();
    float dot = 0.f;
    const KVT *kp = ks + key * G::LDW + half * (HD / 2);
    const float *qp = &qs[wave][half * (HD / 2)];
#pragma unroll
    for (int c = 0; c < HD / 2; c += G::EPC) dot = kdot(kp + c, qp + c, dot);
    dot += __shfl_xor(dot, 32, 64);
    const bool valid = key < n;
    const float s = valid ? dot * scale : -INFINITY;
    const float mnew = fmaxf(m, wave_max(s));
    const float e = valid ? expf(s - mnew) : 0.f;
    const float corr = expf(m - mnew);
    l = l * corr + wave_sum(half ? 0.f : e);
    o0 *= corr;
    o1 *= corr;
    m = mnew;
    if (!half) ps[wave][key] = e;
    __syncthreads();
#pragma unroll 8
    for (int j = 0; j < AT_T; j++) {
      const float ej = ps[wave][j];
      const float2 v = vpair(vs + j * G::LDW + lane * 2);
      o0 = fmaf(ej, v.x, o0);
      o1 = fmaf(ej, v.y, o1);
    }
  }
  out[(size_t)t * QD + h * HD + lane * 2] = o0 / l;
  out[(size_t)t * QD + h * HD + lane * 2 + 1] = o1 / l;
}

}  // namespace vx
