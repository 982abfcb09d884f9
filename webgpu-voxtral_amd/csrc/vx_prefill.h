// vx_prefill.h -- batched prefill of the backbone.  The reference prefills
// one token per backboneStep (src/engine.ts:2457-2472); here a chunk of up
// to PF_MAXT prompt tokens goes through each layer at once, so every weight
// is read once per chunk and the projections are GEMMs
//   C[s][col][m] = sum_{k in slice s} W[m][k] * (B[col][k] + B[nt + col][k])
// (f16 x f16 -> f32 on the matrix cores: vx_gemm.h).  W is the layer's f16
// weight matrix (row-major, as loaded); B holds the chunk's activations in
// hi/lo form (column t = f16(y_t), column nt + t = f16(y_t - hi), each
// column's K halves contiguous), so the product keeps f32 accuracy.  The
// GEMM leaves ns partial sums over slices of K in ns consecutive [nt][ldc]
// blocks of C, and the consumer adds them in order.  Small per-token kernels do RoPE + K/V writes and the causal
// attention, and each of them, or a residual add + RMSNorm, or SwiGLU,
// writes the next GEMM's B directly.  The
// result (K/V cache rows, residual stream, final norm of the last token,
// position) equals that of the per-token steps up to f32 summation order.
#pragma once
#include "vx_kernels.h"
#include <type_traits>

namespace vx {

constexpr int PF_MAXT = 1024;          // tokens per chunk, at most
constexpr int PF_NC = 2 * PF_MAXT;     // B columns (hi, lo), at most
// A chunk of n tokens uses nt = n rounded up to 128 hi columns and as many
// lo columns: N = 2 nt GEMM columns.
__host__ __device__ constexpr int pf_nt(int n) { return (n + 127) / 128 * 128; }

// value of output (token t, row m): the sum of the NS K-slice blocks, in order
template <int NS>
__device__ __forceinline__ float pf_c(const float *C, int ldc, int nt, int t, int m) {
  float v[NS];
#pragma unroll
  for (int s = 0; s < NS; s++) v[s] = C[((size_t)s * nt + t) * ldc + m];
  float y = v[0];
#pragma unroll
  for (int s = 1; s < NS; s++) y += v[s];
  return y;
}
// four consecutive rows m .. m + 3 (m % 4 == 0)
template <int NS>
__device__ __forceinline__ f32x4 pf_c4(const float *C, int ldc, int nt, int t, int m) {
  f32x4 v[NS];
#pragma unroll
  for (int s = 0; s < NS; s++) v[s] = *(const f32x4 *)(C + ((size_t)s * nt + t) * ldc + m);
  f32x4 y = v[0];
#pragma unroll
  for (int s = 1; s < NS; s++) y += v[s];
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

// B columns t and nt + t (K halves each) from row t of X, optionally
// RMS-normalised with gains g (rmsNorm, src/shaders.ts:137-183); columns of
// tokens t >= n are zero.  Grid: nt blocks of 256.
template <bool NORM>
__global__ __launch_bounds__(256) void pf_pack_kernel(const float *X, int K, int n, int nt,
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
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const int k = kb * 8 + e;
      y[e] = t < n ? (NORM ? x[k] * r * h2f(g[k]) : x[k]) : 0.f;
    }
    split_n<8>(y, hi, lo);
    B[(size_t)t * (K / 8) + kb] = hi;
    B[(size_t)(nt + t) * (K / 8) + kb] = lo;
  }
}

// QKV outputs: interleaved rope of q and k at position pos0 + t
// (src/shaders.ts:224-256), q -> Q[t][QD], k and v -> cache rows pos0 + t.
// Grid: (n, QKV_ROWS / 2 / 256), one row pair per thread.
template <int NS>
__global__ void pf_qkv_epi_kernel(const float *C, int nt, float *Q, void *kc, void *vc, int kv_f32,
                                  int max_seq, int pos0, const float *inv_freq) {
  const int t = blockIdx.x, row = 2 * (blockIdx.y * blockDim.x + threadIdx.x);
  const float y0 = pf_c<NS>(C, QKV_ROWS, nt, t, row), y1 = pf_c<NS>(C, QKV_ROWS, nt, t, row + 1);
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

// hi/lo halves of y into B columns t and nt + t at k (8 consecutive k)
__device__ __forceinline__ void pf_put8(h8 *B, int K, int nt, int t, int kb, const float (&y)[8]) {
  h8 hi, lo;
  split_n<8>(y, hi, lo);
  B[(size_t)t * (K / 8) + kb] = hi;
  B[(size_t)(nt + t) * (K / 8) + kb] = lo;
}

// Residual add of a DIM-row GEMM output, X[t] += y (addInPlace,
// src/shaders.ts:532-547), then, with PACK, the next GEMM's B from
// rmsNorm(X[t]) * g (src/shaders.ts:137-183); columns of tokens t >= n are
// zero.  Grid: nt blocks (n without PACK) of 256; thread i owns the 8-value
// groups i and i + 256 (DIM / 8 = 384 groups).
template <bool PACK, int NS>
__global__ __launch_bounds__(256) void pf_resid_pack_kernel(const float *C, int n, int nt, float *X,
                                                            const uint16_t *g, float eps, h8 *B) {
  constexpr int NG = DIM / 8, GPT = (NG + 255) / 256;
  const int t = blockIdx.x, tid = threadIdx.x;
  float v[GPT][8];
  float ss = 0.f;
  if (t < n) {
#pragma unroll
    for (int i = 0; i < GPT; i++) {
      const int kb = tid + 256 * i;
      if (kb < NG) {
        float *x = X + (size_t)t * DIM + kb * 8;
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const f32x4 xv = *(const f32x4 *)(x + 4 * h), a = pf_c4<NS>(C, DIM, nt, t, kb * 8 + 4 * h);
#pragma unroll
          for (int e = 0; e < 4; e++) v[i][4 * h + e] = xv[e] + a[e];
          *(f32x4 *)(x + 4 * h) = f32x4{v[i][4 * h], v[i][4 * h + 1], v[i][4 * h + 2], v[i][4 * h + 3]};
        }
#pragma unroll
        for (int e = 0; e < 8; e++) ss = fmaf(v[i][e], v[i][e], ss);
      }
    }
  }
  if (!PACK) return;
  float r = 0.f;
  if (t < n) {
    __shared__ float red[4];
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    r = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)DIM + eps);
  }
#pragma unroll
  for (int i = 0; i < GPT; i++) {
    const int kb = tid + 256 * i;
    if (kb < NG) {
      float y[8];
#pragma unroll
      for (int e = 0; e < 8; e++) y[e] = t < n ? v[i][e] * r * h2f(g[kb * 8 + e]) : 0.f;
      pf_put8(B, DIM, nt, t, kb, y);
    }
  }
}

// SwiGLU of the stacked [W1; W3] output (ldc = 2 HID; swiGLU,
// src/shaders.ts:483-501) written as the down GEMM's B (K = HID); columns of
// tokens t >= n are zero.  Grid: (nt, HID / 8 / 128) of 128, one 8-value
// group per thread.
template <int NS>
__global__ __launch_bounds__(128) void pf_swiglu_pack_kernel(const float *C, int n, int nt, h8 *B) {
  const int t = blockIdx.x, kb = blockIdx.y * 128 + threadIdx.x;
  float y[8];
  if (t < n) {
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const f32x4 gt = pf_c4<NS>(C, 2 * HID, nt, t, kb * 8 + 4 * h);
      const f32x4 up = pf_c4<NS>(C, 2 * HID, nt, t, HID + kb * 8 + 4 * h);
#pragma unroll
      for (int e = 0; e < 4; e++) y[4 * h + e] = (gt[e] / (1.0f + expf(-gt[e]))) * up[e];
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; e++) y[e] = 0.f;
  }
  pf_put8(B, HID, nt, t, kb, y);
}
static_assert(DIM % 8 == 0 && (HID / 8) % 128 == 0, "prefill packing groups");

// ------------------------------------------------ causal attention on MFMA
// Causal attention of the chunk (attnScore + softmax + attnValue per prompt
// token over keys 0..pos0+t, src/shaders.ts:306-447) with the products on the
// matrix cores; blocks of tokens t >= n write zero columns of the O GEMM's B.
// Block = (16-token tile, KV head) of PFA_KG groups of 4 waves; wave w of a
// group is query head 4*kv_head + w.  The tile's keys are taken 32 at a
// time: group g stages tiles g, g + PFA_KG, ... in its own LDS area, K rows
// and transposed V rows already split into f16 hi and lo (once per group,
// not once per wave), shared by its 4 waves, and keeps its own online
// softmax; the groups' (max, sum, O) are merged through LDS at the end.
// Per 32-key tile and wave, in the transposed form (the token is the MFMA
// column, so every lane holds one token's values):
//   S^T[16 keys][16 tokens] = K[16][128] . Q^T[128][16]     16x16x32 f16
//   O^T[16 dims][16 tokens] += V^T[16][16 keys] . P^T[16 keys][16]   16x16x16 f16
// The D layout of S^T (lane l: keys 4(l/16)..+3 of token l%16) is exactly
// the B operand of the 16x16x16 product, so P needs no shuffle; the online
// softmax rescale of O^T is per lane.  Every f32 operand is split into f16
// hi + lo and a product is hi.hi + hi.lo + lo.hi, about 2^-20 relative (the
// dropped lo.lo term), where the prefill GEMMs, with exact f16 weights, are
// at the split's 2^-21.  An f16 cache is exact in f16: its lo halves are
// zero, so they are neither stored nor multiplied.  Output: hi/lo
// rows of the O projection's B (rows t and nt + t), zero for t >= n.
typedef _Float16 hf4 __attribute__((ext_vector_type(4)));
constexpr int PFA_T = 16;          // tokens per block
constexpr int PFA_K = 32;          // keys per staged tile
constexpr int PFA_KW = HD + 8;     // LDS row of K, halves (272 B)
constexpr int PFA_VW = PFA_K + 4;  // LDS row of V^T, halves (72 B: 16 rows start on 16 distinct even banks)
constexpr int PFA_KG = 2;          // key groups per block
constexpr int PFA_GROUP = 2 * (PFA_K * PFA_KW + HD * PFA_VW);  // halves of one group's area (hi + lo)
constexpr int PFA_LDS = PFA_KG * PFA_GROUP * 2;                // dynamic LDS bytes (70 KB)
constexpr int PFA_RED = 2 + 4 * (HD / 16);                     // merged values per lane: m, l, O^T
static_assert((PFA_KG - 1) * 4 * PFA_RED * 64 * 4 <= PFA_LDS, "merge area");

// hi/lo operand halves (split2) of 8 or 4 f32 values
__device__ __forceinline__ void split8(const f32x4 a, const f32x4 b, h8 &hi, h8 &lo) {
  const float x[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  split_n<8>(x, hi, lo);
}
__device__ __forceinline__ void split4(const f32x4 a, hf4 &hi, hf4 &lo) {
  const float x[4] = {a[0], a[1], a[2], a[3]};
  split_n<4>(x, hi, lo);
}

// 4 consecutive K/V values as held between load and staging: f32 as loaded,
// f16 as raw halves (widened only when staged, so the prefetch's wait stays
// at the staging point)
__device__ __forceinline__ f32x4 pfa_ld4(const float *p) { return *(const f32x4 *)p; }
__device__ __forceinline__ uint2 pfa_ld4(const uint16_t *p) { return *(const uint2 *)p; }
__device__ __forceinline__ f32x4 pfa_widen(f32x4 v) { return v; }
__device__ __forceinline__ f32x4 pfa_widen(uint2 v) {
  const h2 a = __builtin_bit_cast(h2, v.x), b = __builtin_bit_cast(h2, v.y);
  return f32x4{(float)a.x, (float)a.y, (float)b.x, (float)b.y};
}

// KVT = float (f32 cache) or uint16_t (f16 cache).
// Launch: grid (nt / PFA_T, NKV), 256 * PFA_KG threads, PFA_LDS dynamic LDS.
template <typename KVT>
__global__ __launch_bounds__(256 * PFA_KG) void pf_attn_mfma_kernel(const float *Q, const KVT *kc,
                                                                    const KVT *vc, int max_seq, int pos0,
                                                                    int n, int nt, h8 *B) {
  constexpr bool EXACT = std::is_same<KVT, uint16_t>::value;  // f16 cache: no lo halves
  extern __shared__ __attribute__((aligned(16))) _Float16 pfa_smem[];
  const int t0 = blockIdx.x * PFA_T, kvh = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int grp_k = wave >> 2, hw = wave & 3;  // key group, head within the KV group
  const int h = kvh * (NH / NKV) + hw;
  const int col = lane & 15, grp = lane >> 4;  // MFMA column (token) and row group
  const int t = t0 + col;                      // this lane's token
  _Float16 *khs = pfa_smem + grp_k * PFA_GROUP, *kls = khs + PFA_K * PFA_KW;
  _Float16 *vhs = kls + PFA_K * PFA_KW, *vls = vhs + HD * PFA_VW;
  if (t0 >= n) {  // padding columns of the GEMM: zero hi and lo (group 0 writes)
    if (grp_k == 0) {
      _Float16 *p = (_Float16 *)B;
#pragma unroll
      for (int dt = 0; dt < HD / 16; dt++) {
        const size_t c = (size_t)h * HD + dt * 16 + 4 * grp;
        *(hf4 *)(p + (size_t)t * QD + c) = hf4{0, 0, 0, 0};
        *(hf4 *)(p + (size_t)(nt + t) * QD + c) = hf4{0, 0, 0, 0};
      }
    }
    return;
  }
  const KVT *Kb = kc + (size_t)kvh * max_seq * HD;
  const KVT *Vb = vc + (size_t)kvh * max_seq * HD;
  const int last = pos0 + min(t, n - 1);         // last key of this lane's token
  const int kend = pos0 + min(t0 + PFA_T, n);    // keys of the tile: [0, kend)
  const int ntile = (kend + PFA_K - 1) / PFA_K;
  const int iters = (ntile + PFA_KG - 1) / PFA_KG;  // the same count in every group

  // staging, thread i of its group: K rows (i / 32) + 8j, dims 4 (i % 32)
  // (row-major LDS writes); V keys 2 (i % 16) and 2 (i % 16) + 1, dims
  // 4 (i / 16) and 64 + 4 (i / 16), so each transposed LDS write holds the
  // pair of keys as one dword
  const int gtid = tid & 255, srow = gtid >> 5, sdim = (gtid & 31) * 4;
  const int vkey = 2 * (gtid & 15), vdim = 4 * (gtid >> 4);
  decltype(pfa_ld4(Kb)) kr[4], vr[4];
  auto load_tile = [&](int kb) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int key = min(kb + srow + 8 * j, kend - 1);  // rows past the keys re-read the last
      kr[j] = pfa_ld4(Kb + (size_t)key * HD + sdim);
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {  // vr[j]: key vkey + (j >> 1), dims vdim + 64 (j & 1)
      const int key = min(kb + vkey + (j >> 1), kend - 1);
      vr[j] = pfa_ld4(Vb + (size_t)key * HD + vdim + 64 * (j & 1));
    }
  };
  if (grp_k < ntile) load_tile(grp_k * PFA_K);

  // Q^T operand of S^T (token t, dims 32c + 8grp..+8), hi and lo; padding tokens zero
  h8 qh[HD / 32], ql[HD / 32];
  {
    const float *qp = Q + (size_t)min(t, n - 1) * QD + h * HD + 8 * grp;
#pragma unroll
    for (int c = 0; c < HD / 32; c++) {
      f32x4 a = *(const f32x4 *)(qp + 32 * c), b = *(const f32x4 *)(qp + 32 * c + 4);
      if (t >= n) a = b = f32x4{0.f, 0.f, 0.f, 0.f};
      split8(a, b, qh[c], ql[c]);
    }
  }
  const float scale = 1.0f / sqrtf((float)HD);
  float m = -INFINITY, l = 0.f;
  f32x4 o[HD / 16];
#pragma unroll
  for (int dt = 0; dt < HD / 16; dt++) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int i = 0; i < iters; i++) {
    const int it = grp_k + PFA_KG * i, kb = it * PFA_K;
    const bool live = it < ntile;  // uniform over the group
    __syncthreads();  // the previous tile's LDS reads are done
    if (live) {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        hf4 hi, lo;
        split4(pfa_widen(kr[j]), hi, lo);
        *(hf4 *)(khs + (srow + 8 * j) * PFA_KW + sdim) = hi;
        if (!EXACT) *(hf4 *)(kls + (srow + 8 * j) * PFA_KW + sdim) = lo;
      }
#pragma unroll
      for (int hd = 0; hd < 2; hd++) {
        const f32x4 va = pfa_widen(vr[hd]), vb = pfa_widen(vr[2 + hd]);  // keys vkey, vkey + 1
#pragma unroll
        for (int q = 0; q < 4; q++) {
          h2 hi, lo;
          split2(va[q], vb[q], hi, lo);
          const int d = vdim + 64 * hd + q;
          *(h2 *)(vhs + d * PFA_VW + vkey) = hi;
          if (!EXACT) *(h2 *)(vls + d * PFA_VW + vkey) = lo;
        }
      }
      if (it + PFA_KG < ntile) load_tile(kb + PFA_KG * PFA_K);
    }
    __syncthreads();
    if (!live) continue;

    // S^T for keys kb + 16kt + (4grp..+3), token col
    f32x4 s[2];
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
      f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
      const int ro = (16 * kt + col) * PFA_KW + 8 * grp;
#pragma unroll
      for (int c = 0; c < HD / 32; c++) {
        const h8 kh = *(const h8 *)(khs + ro + 32 * c);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[c], acc, 0, 0, 0);
        if (!EXACT) {
          const h8 kl = *(const h8 *)(kls + ro + 32 * c);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qh[c], acc, 0, 0, 0);
        }
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql[c], acc, 0, 0, 0);
      }
      s[kt] = acc;
    }
    // online softmax of token col over this tile's keys (8 per lane, 4 lanes per token)
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int key = kb + 16 * kt + 4 * grp + q;
        const float v = key <= last ? s[kt][q] * scale : -INFINITY;
        s[kt][q] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    // a token whose keys all lie past this tile's start keeps m = -inf
    // (only in groups other than 0: key 0 <= last is in tile 0)
    const float mnew = fmaxf(m, mx);
    const float corr = mnew == -INFINITY ? 1.0f : expf(m - mnew);
    float ps = 0.f;
#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const float e = s[kt][q] == -INFINITY ? 0.f : expf(s[kt][q] - mnew);
        s[kt][q] = e;
        ps += e;
      }
    ps += __shfl_xor(ps, 16, 64);
    ps += __shfl_xor(ps, 32, 64);
    l = l * corr + ps;
    m = mnew;
    // O^T += V^T . P^T
    hf4 ph[2], pl[2];
#pragma unroll
    for (int kt = 0; kt < 2; kt++) split4(s[kt], ph[kt], pl[kt]);
#pragma unroll
    for (int dt = 0; dt < HD / 16; dt++) {
      f32x4 acc = o[dt] * corr;
#pragma unroll
      for (int kt = 0; kt < 2; kt++) {
        const int ro = (16 * dt + col) * PFA_VW + 16 * kt + 4 * grp;
        const hf4 vh = *(const hf4 *)(vhs + ro);
        acc = __builtin_amdgcn_mfma_f32_16x16x16f16(vh, ph[kt], acc, 0, 0, 0);
        if (!EXACT) {
          const hf4 vl = *(const hf4 *)(vls + ro);
          acc = __builtin_amdgcn_mfma_f32_16x16x16f16(vl, ph[kt], acc, 0, 0, 0);
        }
        acc = __builtin_amdgcn_mfma_f32_16x16x16f16(vh, pl[kt], acc, 0, 0, 0);
      }
      o[dt] = acc;
    }
  }
  // merge the groups' (m, l, O^T) in group order: groups 1.. write theirs
  // to LDS (lane-minor), group 0 combines them
  if (PFA_KG > 1) {
    float *red = (float *)pfa_smem;
    __syncthreads();  // every group is done with its staging area
    if (grp_k > 0) {
      float *r = red + ((grp_k - 1) * 4 + hw) * PFA_RED * 64 + lane;
      r[0] = m;
      r[64] = l;
#pragma unroll
      for (int dt = 0; dt < HD / 16; dt++)
#pragma unroll
        for (int q = 0; q < 4; q++) r[(2 + 4 * dt + q) * 64] = o[dt][q];
    }
    __syncthreads();
    if (grp_k > 0) return;
    float mg[PFA_KG];
    mg[0] = m;
#pragma unroll
    for (int g = 1; g < PFA_KG; g++) mg[g] = red[((g - 1) * 4 + hw) * PFA_RED * 64 + lane];
    float mm = mg[0];
#pragma unroll
    for (int g = 1; g < PFA_KG; g++) mm = fmaxf(mm, mg[g]);
    const float c0 = expf(m - mm);  // m is finite in group 0
    l *= c0;
#pragma unroll
    for (int dt = 0; dt < HD / 16; dt++) o[dt] = o[dt] * c0;
#pragma unroll
    for (int g = 1; g < PFA_KG; g++) {
      const float *rg = red + ((g - 1) * 4 + hw) * PFA_RED * 64 + lane;
      const float cg = mg[g] == -INFINITY ? 0.f : expf(mg[g] - mm);
      l += rg[64] * cg;
#pragma unroll
      for (int dt = 0; dt < HD / 16; dt++)
#pragma unroll
        for (int q = 0; q < 4; q++) o[dt][q] += rg[(2 + 4 * dt + q) * 64] * cg;
    }
  }
  // out[t][dims] = O^T / l, as hi and lo f16 rows of B (zero past n)
  _Float16 *p = (_Float16 *)B;
  const float inv = 1.0f / l;
#pragma unroll
  for (int dt = 0; dt < HD / 16; dt++) {
    hf4 hi = hf4{0, 0, 0, 0}, lo = hf4{0, 0, 0, 0};
    if (t < n) split4(o[dt] * inv, hi, lo);
    const size_t c = (size_t)h * HD + dt * 16 + 4 * grp;
    *(hf4 *)(p + (size_t)t * QD + c) = hi;
    *(hf4 *)(p + (size_t)(nt + t) * QD + c) = lo;
  }
}

}  // namespace vx
