// vx_kernels.h -- HIP kernels of the MI355X (gfx950) Voxtral frame loop.
//
// Device layout (all in HBM, owned by the engine):
//   weights   f16 row-major [out][in]; per backbone layer the Q, K and V
//             projections are stacked into one [6144][3072] matrix.
//   KV cache  f16 [layer][K|V][kv_head][max_seq][128] (head-major, so one
//             split of one KV head reads a contiguous run of rows).
//   activations f32.
//
// Kernels (each replaces one or more WGSL shaders of src/shaders.ts):
//   gemv_kernel      matvecF16 (:21-71) and its Offset/Chunked forms, with
//                    fused prologue (rmsNorm :137-183) and epilogues (rope
//                    :224-256 + kvCacheWrite :452-473; addInPlace :532-547;
//                    swiGLU :483-501).  NB input vectors share each weight
//                    read (NB = 6 for the CFG-batched FM).
//   attn_decode_kernel  attnScore/softmax/attnValue (:306-447) as split-K
//                    flash decoding with a last-block log-sum-exp combine.
//   fm_* kernels     biAttn* (:684-807), timeEmbedding (:579-602),
//                    cfgCombine/eulerStep (:611-648), fsqQuantize (:653-673).
//   argmax_kernel    argmax (:1154-1211), same 256-lane tree tie rule.
//   embed kernels    embeddingLookup (:193-213), multiCodebookEmbed
//                    (:1878-1917).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vx {

constexpr int DIM = 3072;
constexpr int HD = 128;
constexpr int NH = 32;
constexpr int NKV = 8;
constexpr int QD = NH * HD;    // 4096
constexpr int KVD = NKV * HD;  // 1024
constexpr int HID = 9216;
constexpr int QKV_ROWS = QD + 2 * KVD;  // 6144
constexpr int NAC = 36;
constexpr int SEMV = 8320;
// Decode attention is split over the key axis: ATTN_SPLITS blocks per KV
// head, each taking ceil(keys / ATTN_SPLITS) keys.
constexpr int ATTN_SPLITS = 32;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// 16 bytes of a weight matrix.  Weights are read once per pass, so the
// loads carry the non-temporal hint (global_load_dwordx4 ... nt): on MI355X
// these stream faster than plain loads and neither allocate in nor evict
// from the memory-side Infinity Cache.
__device__ __forceinline__ u32x4 ldw(const void *p) { return __builtin_nontemporal_load((const u32x4 *)p); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
// The same sum without the LDS crossbar: four DPP steps leave each row of 16
// lanes holding its row sum (quad_perm xor 1, xor 2, half-row mirror, row
// mirror), then the four row sums are read out and added in a fixed order.
// Every lane gets the same value.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_mov<0x141>(v);  // row_half_mirror
  v += dpp_mov<0x140>(v);  // row_mirror
  const int b = __builtin_bit_cast(int, v);
  return (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16))) +
         (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48)));
}
// maximum over the wave by the same DPP steps as wave_sum_dpp
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_mov<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_mov<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_mov<0x141>(v));  // row_half_mirror
  v = fmaxf(v, dpp_mov<0x140>(v));  // row_mirror
  const int b = __builtin_bit_cast(int, v);
  return fmaxf(fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)),
                     __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16))),
               fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)),
                     __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48))));
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

__device__ __forceinline__ float h2f(uint16_t b) {
  return (float)__builtin_bit_cast(_Float16, b);
}
__device__ __forceinline__ uint16_t f2h(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);  // v_cvt_f16_f32, RNE
}
// x = hi + lo in f16 for two values: hi = f16(x) rounded toward zero, from
// one v_cvt_pkrtz_f16_f32, and lo = f16(x - hi) rounded to nearest even from
// that same hi, so |x - hi - lo| <= 2^-21 |x| for normal hi (f16 subnormals
// are kept).  The sum is only that close when lo is formed from the very hi
// that is stored.  Written as plain casts, the compiler converts hi twice
// (packed for the stored operand, scalar for the remainder), and the pairing
// then rests on both conversions being generated right; this compiler has
// been seen to emit the packed one with its second source replaced by the
// first.  Inline asm is no way out: the hazard recognizer does not count an
// asm statement as a vector-ALU write, so an MFMA that reads its result gets
// no wait states and reads the register's old contents.
__device__ __forceinline__ void split2(float a, float b, h2 &hi, h2 &lo) {
  const auto h = __builtin_amdgcn_cvt_pkrtz(a, b);
  hi = h2{(_Float16)h[0], (_Float16)h[1]};
  lo = h2{(_Float16)(a - (float)h[0]), (_Float16)(b - (float)h[1])};
}
// split2 over N values (N even) into f16 vectors of N lanes
template <int N, typename V>
__device__ __forceinline__ void split_n(const float (&x)[N], V &hi, V &lo) {
#pragma unroll
  for (int j = 0; j < N; j += 2) {
    h2 h, l;
    split2(x[j], x[j + 1], h, l);
    hi[j] = h[0];
    hi[j + 1] = h[1];
    lo[j] = l[0];
    lo[j + 1] = l[1];
  }
}
// IEEE binary16 round-to-nearest-even in integer arithmetic, subnormals
// included; used where results must be bit-identical to the CPU generator
// whatever the device's float mode.
__device__ __forceinline__ uint16_t f2h_exact(float f) {
  const uint32_t x = __builtin_bit_cast(uint32_t, f);
  const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u)
    return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u | ((ax >> 13) & 0x3ffu) : 0x7c00u));
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
  uint32_t q, rem, half;
  if (ax < 0x38800000u) {  // result is subnormal (or zero): q * 2^-24
    if (ax <= 0x33000000u) return (uint16_t)sign;
    const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    const int rsh = 126 - (int)(ax >> 23);  // 14..24
    q = m >> rsh;
    rem = m & ((1u << rsh) - 1u);
    half = 1u << (rsh - 1);
  } else {
    q = (((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13);
    rem = ax & 0x1fffu;
    half = 0x1000u;
  }
  if (rem > half || (rem == half && (q & 1u))) q++;
  return (uint16_t)(sign | q);
}

// acc += sum_j w[j] * x[j] for 8 halves packed in a u32x4
// (vector elements are copied to scalars first: __builtin_bit_cast of an
// ext-vector element expression such as w.y reads element 0)
__device__ __forceinline__ float dot8(u32x4 w, f32x4 xa, f32x4 xb, float acc) {
  const uint32_t w0 = w[0], w1 = w[1], w2 = w[2], w3 = w[3];
  h2 p0 = __builtin_bit_cast(h2, w0), p1 = __builtin_bit_cast(h2, w1),
     p2 = __builtin_bit_cast(h2, w2), p3 = __builtin_bit_cast(h2, w3);
  acc = fmaf((float)p0.x, xa.x, acc);
  acc = fmaf((float)p0.y, xa.y, acc);
  acc = fmaf((float)p1.x, xa.z, acc);
  acc = fmaf((float)p1.y, xa.w, acc);
  acc = fmaf((float)p2.x, xb.x, acc);
  acc = fmaf((float)p2.y, xb.y, acc);
  acc = fmaf((float)p3.x, xb.z, acc);
  acc = fmaf((float)p3.y, xb.w, acc);
  return acc;
}

// ------------------------------------------------------------------ GEMV
enum Epi : int {
  EPI_PLAIN = 0,   // out[b*os + row] = y
  EPI_RESID = 1,   // out[b*os + row] += y   (residual add)
  EPI_SWIGLU = 2,  // rows come in (W row i, W2 row i) pairs: out = silu(g)*u
  EPI_QKV_ROPE = 3,// backbone: rope q,k at *pos; q -> out, k,v -> f16 cache
  EPI_QKV = 4,     // FM: q -> out, k -> out_k, v -> out_v (no rope)
};

// Launch timeline (vx_debug_timeline): block b of a launch writes its start
// and end time on the 100 MHz wall clock to ts[2 b], ts[2 b + 1] with plain
// vector stores (distinct addresses: no contention); the host takes the
// earliest start and the latest end.  ts is null outside that measurement.
constexpr int TS_BLOCKS = 1024;  // slots per launch (the widest grid is 768 blocks)
__device__ __forceinline__ void ts_begin(unsigned long long *ts) {
  if (ts && threadIdx.x == 0) ts[2 * blockIdx.x] = wall_clock64();
}
__device__ __forceinline__ void ts_end(unsigned long long *ts) {
  if (ts) {
    __syncthreads();
    if (threadIdx.x == 0) ts[2 * blockIdx.x + 1] = wall_clock64();
  }
}

struct GemvArgs {
  const uint16_t *W;   // [M][K]
  const uint16_t *W2;  // SwiGLU up matrix [M][K]
  const float *x;      // NB vectors, vector stride xs
  int xs;
  const uint16_t *norm_w;  // RMSNorm gains (NORM variants)
  float eps;
  float *out;  // output base, vector stride os
  int os;
  float *out_k, *out_v;  // EPI_QKV
  int M;                 // rows (EPI_SWIGLU: row pairs)
  // EPI_QKV_ROPE
  const int *pos;
  void *kc, *vc;  // this layer's K and V cache [NKV][max_seq][HD], f32 or f16
  int kv_f32;     // 1: f32 cache elements (the reference's), 0: f16
  int max_seq;
  const float *inv_freq;  // rope: 1 / theta^(2i/HD), i < HD/2
  unsigned long long *ts;  // launch timeline slot (passed as gemv1_kernel's ts argument), or null
};

// one K/V cache element pair (d, d+1) of head row `row` at position pos
__device__ __forceinline__ void kv_store2(void *cache, int kv_f32, int max_seq, int c, int pos,
                                          float v0, float v1) {
  const size_t off = ((size_t)(c >> 7) * max_seq + pos) * HD + (c & (HD - 1));
  if (kv_f32) {
    float *d = (float *)cache + off;
    d[0] = v0;
    d[1] = v1;
  } else {
    uint16_t *d = (uint16_t *)cache + off;
    d[0] = f2h(v0);
    d[1] = f2h(v1);
  }
}

// Batched GEMV (the FM's CFG batch and the small projections; EPI_QKV_ROPE
// is served by gemv1_kernel).  Rows handled per wave = RPW (EPI_SWIGLU: RPW/2 pairs).  The block stages
// the NB input vectors (RMS-normalised when NORM) into LDS one K-tile of KT
// floats at a time; each lane streams 16-byte weight chunks, chunk c of a
// row covering columns [c*512 + lane*8, +8), so a wave reads 1 KB of one
// row per load instruction.
template <int NB, int WAVES, int RPW, int EPI, bool NORM, int K, int KT>
__global__ __launch_bounds__(WAVES * 64) void gemv_kernel(const uint16_t *W, const uint16_t *W2, const float *x,
                                                         const uint16_t *norm_w, float *out, GemvArgs args) {
  // leading pointer arguments: preloaded into SGPRs (as in gemv1_kernel)
  GemvArgs a = args;
  a.W = W;
  a.W2 = W2;
  a.x = x;
  a.norm_w = norm_w;
  a.out = out;
  static_assert(KT == K && K % 512 == 0 && EPI != EPI_QKV_ROPE, "one K tile");
  constexpr int NT = WAVES * 64;
  constexpr int NCH = K / 512;
  static_assert(K % (NT * 4) == 0, "threads tile K");
  constexpr int XPV = K / (NT * 4);  // float4s of one input vector per thread
  __shared__ __attribute__((aligned(16))) float xl[NB * K];
  __shared__ float red[WAVES][NB];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int unit0 = (blockIdx.x * WAVES + wave) * (EPI == EPI_SWIGLU ? RPW / 2 : RPW);
  const bool active = unit0 < a.M;

  // input vectors (and RMSNorm gains) first, then the weights: per-wave
  // loads return in issue order, so the prologue below waits only on the
  // former while the weights are in flight
  f32x4 xv[NB][XPV];
  uint2 gv[XPV];
#pragma unroll
  for (int i = 0; i < XPV; i++) {
    const int k = (tid + i * NT) * 4;
#pragma unroll
    for (int b = 0; b < NB; b++) xv[b][i] = *(const f32x4 *)(a.x + (size_t)b * a.xs + k);
    if (NORM) gv[i] = *(const uint2 *)(a.norm_w + k);
  }
  u32x4 w[RPW][NCH];
#pragma unroll
  for (int r = 0; r < RPW; r++) {
    const uint16_t *rowp;
    if (EPI == EPI_SWIGLU)
      rowp = ((r & 1) ? a.W2 : a.W) + (size_t)min(unit0 + (r >> 1), a.M - 1) * K;
    else
      rowp = a.W + (size_t)min(unit0 + r, a.M - 1) * K;
#pragma unroll
    for (int c = 0; c < NCH; c++) w[r][c] = ldw(rowp + c * 512 + lane * 8);
  }

  float scl[NB];
#pragma unroll
  for (int b = 0; b < NB; b++) scl[b] = 1.0f;
  if (NORM) {  // rmsNorm prologue: rms = 1/sqrt(mean(x^2) + eps)
#pragma unroll
    for (int b = 0; b < NB; b++) {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < XPV; i++)
        s += xv[b][i].x * xv[b][i].x + xv[b][i].y * xv[b][i].y + xv[b][i].z * xv[b][i].z +
             xv[b][i].w * xv[b][i].w;
      s = wave_sum_dpp(s);
      if (lane == 0) red[wave][b] = s;
    }
    __syncthreads();
#pragma unroll
    for (int b = 0; b < NB; b++) {
      float s = 0.f;
#pragma unroll
      for (int q = 0; q < WAVES; q++) s += red[q][b];
      scl[b] = 1.0f / sqrtf(s / (float)K + a.eps);
    }
  }
#pragma unroll
  for (int i = 0; i < XPV; i++) {
    const int k = (tid + i * NT) * 4;
#pragma unroll
    for (int b = 0; b < NB; b++) {
      f32x4 v = xv[b][i];
      if (NORM) {
        const float r = scl[b];
        const h2 g01 = __builtin_bit_cast(h2, gv[i].x), g23 = __builtin_bit_cast(h2, gv[i].y);
        v.x = v.x * r * (float)g01.x;
        v.y = v.y * r * (float)g01.y;
        v.z = v.z * r * (float)g23.x;
        v.w = v.w * r * (float)g23.y;
      }
      *(f32x4 *)(xl + b * K + k) = v;
    }
  }
  __syncthreads();

  float acc[RPW][NB];
#pragma unroll
  for (int r = 0; r < RPW; r++)
#pragma unroll
    for (int b = 0; b < NB; b++) acc[r][b] = 0.f;
  if (active) {
#pragma unroll
    for (int c = 0; c < NCH; c++)
#pragma unroll
      for (int b = 0; b < NB; b++) {
        const float *xp = xl + b * K + c * 512 + lane * 8;
        f32x4 xa = *(const f32x4 *)xp, xb = *(const f32x4 *)(xp + 4);
#pragma unroll
        for (int r = 0; r < RPW; r++) acc[r][b] = dot8(w[r][c], xa, xb, acc[r][b]);
      }
  }
  if (!active) return;

#pragma unroll
  for (int r = 0; r < RPW; r++)
#pragma unroll
    for (int b = 0; b < NB; b++) acc[r][b] = wave_sum_dpp(acc[r][b]);
  if (lane != 0) return;

  if (EPI == EPI_SWIGLU) {
#pragma unroll
    for (int r = 0; r < RPW; r += 2) {
      int i = unit0 + r / 2;
#pragma unroll
      for (int b = 0; b < NB; b++) {
        float g = acc[r][b], u = acc[r + 1][b];
        float silu = g / (1.0f + expf(-g));
        a.out[(size_t)b * a.os + i] = silu * u;
      }
    }
  } else {
#pragma unroll
    for (int r = 0; r < RPW; r++) {
      int row = unit0 + r;
      if (row >= a.M) break;
#pragma unroll
      for (int b = 0; b < NB; b++) {
        float y = acc[r][b];
        if (EPI == EPI_PLAIN) {
          a.out[(size_t)b * a.os + row] = y;
        } else if (EPI == EPI_RESID) {
          float *o = a.out + (size_t)b * a.os + row;
          *o = y + *o;
        } else {  // EPI_QKV
          if (row < QD)
            a.out[(size_t)b * QD + row] = y;
          else if (row < QD + KVD)
            a.out_k[(size_t)b * KVD + row - QD] = y;
          else
            a.out_v[(size_t)b * KVD + row - QD - KVD] = y;
        }
      }
    }
  }
}

// ------------------------------------------------- streaming GEMV (batch 1)
// The backbone GEMVs.  Block b owns units [b*WAVES*UPW, (b+1)*WAVES*UPW) and
// wave w a contiguous run of UPW units, processed in groups of UPG units.  A
// unit is one output row, or a row pair for EPI_SWIGLU (gate row i, up row
// i) and EPI_QKV_ROPE (rows 2i, 2i+1).  Per-wave loads return in issue
// order, so the block first issues its share of the input vector (and the
// RMSNorm gains), then the weight loads of the first D groups; the
// normalised vector is staged into LDS while the weights are in flight, and
// group g+D is issued as soon as group g has been consumed.
template <int EPI>
constexpr int rows_per_unit() {
  return (EPI == EPI_SWIGLU || EPI == EPI_QKV_ROPE) ? 2 : 1;
}

template <int EPI, int K>
__device__ __forceinline__ const uint16_t *unit_row(const GemvArgs &a, int unit, int r) {
  if (EPI == EPI_SWIGLU) return (r ? a.W2 : a.W) + (size_t)unit * K;
  if (EPI == EPI_QKV_ROPE) return a.W + (size_t)(2 * unit + r) * K;
  return a.W + (size_t)unit * K;
}

template <int EPI, int K, int UPG>
__device__ __forceinline__ void load_group(const GemvArgs &a, int unit0, int lane,
                                           u32x4 (&w)[UPG * rows_per_unit<EPI>()][K / 512]) {
  constexpr int RU = rows_per_unit<EPI>();
#pragma unroll
  for (int u = 0; u < UPG; u++)
#pragma unroll
    for (int r = 0; r < RU; r++) {
      const uint16_t *p = unit_row<EPI, K>(a, unit0 + u, r) + lane * 8;
#pragma unroll
      for (int c = 0; c < K / 512; c++) w[u * RU + r][c] = ldw(p + c * 512);
    }
}

// epilogue of one unit; y[r] = full dot product of the unit's row r
template <int EPI>
__device__ __forceinline__ void unit_epilogue(const GemvArgs &a, int unit, const float *y, int pos,
                                              float resid) {
  if (EPI == EPI_SWIGLU) {
    const float g = y[0];
    a.out[unit] = (g / (1.0f + expf(-g))) * y[1];
  } else if (EPI == EPI_QKV_ROPE) {
    const int row = 2 * unit;
    const float y0 = y[0], y1 = y[1];
    if (row < QD + KVD) {
      const int pair = (row & (HD - 1)) >> 1;
      const float freq = a.inv_freq[pair];
      const float ang = (float)pos * freq;
      const float cs = cosf(ang), sn = sinf(ang);
      const float r0 = y0 * cs - y1 * sn, r1 = y0 * sn + y1 * cs;
      if (row < QD) {
        a.out[row] = r0;
        a.out[row + 1] = r1;
      } else {
        kv_store2(a.kc, a.kv_f32, a.max_seq, row - QD, pos, r0, r1);
      }
    } else {
      kv_store2(a.vc, a.kv_f32, a.max_seq, row - QD - KVD, pos, y0, y1);
    }
  } else if (EPI == EPI_RESID) {
    a.out[unit] = y[0] + resid;
  } else {
    a.out[unit] = y[0];
  }
}

template <int WAVES, int UPW, int UPG, int EPI, bool NORM, int K, int D>
__global__ __launch_bounds__(WAVES * 64) void gemv1_kernel(const uint16_t *W, const uint16_t *W2, const float *x,
                                                          const uint16_t *norm_w, float *out,
                                                          unsigned long long *ts, GemvArgs args) {
  ts_begin(ts);
  // the pointers the first loads need arrive as leading scalar arguments,
  // which the hardware preloads into SGPRs at wave launch (no kernel-
  // argument load before the first weight load)
  GemvArgs a = args;
  a.W = W;
  a.W2 = W2;
  a.x = x;
  a.norm_w = norm_w;
  a.out = out;
  constexpr int RU = rows_per_unit<EPI>();
  constexpr int RG = UPG * RU;  // rows per group
  constexpr int NCH = K / 512;
  constexpr int G = UPW / UPG;
  constexpr int NT = WAVES * 64;
  constexpr int XPT = (K + NT * 4 - 1) / (NT * 4);  // input float4s per thread
  constexpr int DD = D < G ? D : G;                  // groups in flight
  static_assert(K % 512 == 0 && UPW % UPG == 0 && D >= 1, "shape");
  __shared__ __attribute__((aligned(16))) float xl[K];
  __shared__ float red[WAVES];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int u0 = (blockIdx.x * WAVES + wave) * UPW;

  // the residual values are read first of all, so the epilogue waits on none
  float resid[UPW];
#pragma unroll
  for (int u = 0; u < UPW; u++) resid[u] = EPI == EPI_RESID ? a.out[u0 + u] : 0.f;
  // when the threads tile K exactly the guard is known true at compile
  // time: an unconditional load lets the compiler issue the weight loads
  // right behind it instead of waiting on it inside a branch
  constexpr bool XEXACT = K % (NT * 4) == 0;
  f32x4 xv[XPT];
  uint2 gv[XPT];
#pragma unroll
  for (int i = 0; i < XPT; i++) {
    const int k = (tid + i * NT) * 4;
    if (XEXACT || k < K) {
      xv[i] = *(const f32x4 *)(a.x + k);
      if (NORM) gv[i] = *(const uint2 *)(a.norm_w + k);
    }
  }
  u32x4 wbuf[DD][RG][NCH];
#pragma unroll
  for (int g = 0; g < DD; g++) load_group<EPI, K, UPG>(a, u0 + g * UPG, lane, wbuf[g]);

  // stage the input vector (RMSNorm'd: x * rms * w) while the weights fly
  float scale = 1.0f;
  if (NORM) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < XPT; i++)
      if (XEXACT || (tid + i * NT) * 4 < K)
        s += xv[i].x * xv[i].x + xv[i].y * xv[i].y + xv[i].z * xv[i].z + xv[i].w * xv[i].w;
    s = wave_sum_dpp(s);
    if (lane == 0) red[wave] = s;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < WAVES; w++) tot += red[w];
    scale = 1.0f / sqrtf(tot / (float)K + a.eps);
  }
#pragma unroll
  for (int i = 0; i < XPT; i++) {
    const int k = (tid + i * NT) * 4;
    if (XEXACT || k < K) {
      f32x4 v = xv[i];
      if (NORM) {
        const h2 g01 = __builtin_bit_cast(h2, gv[i].x), g23 = __builtin_bit_cast(h2, gv[i].y);
        v.x = v.x * scale * (float)g01.x;
        v.y = v.y * scale * (float)g01.y;
        v.z = v.z * scale * (float)g23.x;
        v.w = v.w * scale * (float)g23.y;
      }
      *(f32x4 *)(xl + k) = v;
    }
  }
  __syncthreads();
  const int pos = (EPI == EPI_QKV_ROPE) ? *a.pos : 0;

#pragma unroll
  for (int g = 0; g < G; g++) {
    float acc[RG];
#pragma unroll
    for (int r = 0; r < RG; r++) acc[r] = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; c++) {
      const float *xp = xl + c * 512 + lane * 8;
      const f32x4 xa = *(const f32x4 *)xp, xb = *(const f32x4 *)(xp + 4);
#pragma unroll
      for (int r = 0; r < RG; r++) acc[r] = dot8(wbuf[g % DD][r][c], xa, xb, acc[r]);
    }
    if (g + DD < G) load_group<EPI, K, UPG>(a, u0 + (g + DD) * UPG, lane, wbuf[g % DD]);
#pragma unroll
    for (int r = 0; r < RG; r++) acc[r] = wave_sum_dpp(acc[r]);
    if (lane == 0) {
#pragma unroll
      for (int u = 0; u < UPG; u++)
        unit_epilogue<EPI>(a, u0 + g * UPG + u, acc + u * RU, pos, resid[g * UPG + u]);
    }
  }
  ts_end(ts);
}

// ------------------------------------------------------ decode attention
struct AttnArgs {
  const float *q;   // [NH*HD], roped
  const void *kc;   // this layer's K cache [NKV][max_seq][HD] (f32 or f16)
  const void *vc;
  const int *pos;   // decode position; keys 0..pos
  int max_seq;
  float *part;      // [NH][ATTN_SPLITS][HD + 2] (o, m, l)
  float *out;       // [NH*HD]
  unsigned long long *ts;  // launch timeline slot (passed as the kernel's ts argument), or null
};

constexpr int AT_T = 32;  // keys per LDS tile

// keys per split for seq keys
__device__ __forceinline__ int attn_chunk(int seq) { return (seq + ATTN_SPLITS - 1) / ATTN_SPLITS; }

// One K or V tile of AT_T key rows in LDS, filled by direct global->LDS
// loads (global_load_lds_dwordx4: 64 lanes x 16 bytes = one 1 KB block per
// instruction, no registers, no staging stores).  Chunk c (16 bytes) of tile
// row r sits at position c ^ kv_sw(r) of its LDS row: the lanes of one score
// read (keys 0..7 x both halves, see the partial kernel) then hit 16
// distinct 16-byte bank groups, and a row read for the value product is a
// permutation of the row.
template <typename KVT>
struct KvRing {
  static constexpr int RB = HD * (int)sizeof(KVT);  // bytes per key row
  static constexpr int CPR = RB / 16;               // 16-byte chunks per row
  static constexpr int RPB = 1024 / RB;             // rows per 1 KB load
  static constexpr int TB = AT_T * RB;              // bytes of one K (or V) tile
  static constexpr int BPT = TB / 1024;             // 1 KB loads per K tile
  static constexpr int LPW = BPT / 2;               // loads per wave per tile (K and V)
  static constexpr int EPC = 16 / (int)sizeof(KVT);
  static constexpr int STAGES = 2;                  // tile t + 1 loads while tile t is used
  static constexpr int LDS = 2048 + STAGES * 2 * TB;  // query heads + K|V stages
};
__device__ __forceinline__ int kv_sw(int r) { return (2 * r) & 15; }

__device__ __forceinline__ void lds_dma16(const void *src, unsigned char *lds) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)lds, 16, 0, 0);
}
// s_waitcnt immediate for vmcnt(vm), the other counters left open
constexpr int attn_vmcnt(int vm) { return (vm & 15) | ((vm >> 4) << 14) | (7 << 4) | (15 << 8); }
// block barrier for LDS only: waits for this wave's LDS reads, not for its
// direct loads in flight (a __syncthreads fence would drain those too)
__device__ __forceinline__ void attn_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

// sum over 16 bytes of K elements times 16/sizeof(KVT) query values
__device__ __forceinline__ float kdot(const float *k, const float *q, float acc) {
  const f32x4 kv = *(const f32x4 *)k, qv = *(const f32x4 *)q;
  acc = fmaf(kv.x, qv.x, acc);
  acc = fmaf(kv.y, qv.y, acc);
  acc = fmaf(kv.z, qv.z, acc);
  return fmaf(kv.w, qv.w, acc);
}
__device__ __forceinline__ float kdot(const uint16_t *k, const float *q, float acc) {
  return dot8(*(const u32x4 *)k, *(const f32x4 *)q, *(const f32x4 *)(q + 4), acc);
}
// two consecutive V elements as floats (scalar loads: the compiler pairs
// them, and keeps them free of a wait on the direct loads still in flight)
__device__ __forceinline__ float2 vpair(const float *v) { return make_float2(v[0], v[1]); }
__device__ __forceinline__ float2 vpair(const uint16_t *v) {
  const h2 p = __builtin_bit_cast(h2, *(const uint32_t *)v);
  return make_float2((float)p.x, (float)p.y);
}
// maximum over the wave when lanes 2k and 2k+1 hold the same value: three DPP
// steps leave each row of 16 lanes holding its maximum, then the four rows
__device__ __forceinline__ float wave_max_pairs(float v) {
  v = fmaxf(v, dpp_mov<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_mov<0x141>(v));  // row_half_mirror
  v = fmaxf(v, dpp_mov<0x140>(v));  // row_mirror
  const int b = __builtin_bit_cast(int, v);
  return fmaxf(fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)),
                     __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16))),
               fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)),
                     __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48))));
}

// Partials (attnScore + softmax + attnValue, src/shaders.ts:306-447, split
// over the key axis): 1-D grid of ATTN_SPLITS * NKV blocks of 256 threads,
// block b = split * NKV + kv head.  Workgroups are dealt to the 8 XCDs
// round-robin, so a KV head's splits (and the combine blocks of its query
// heads) run on one XCD.  Wave w is query head 4*kv_head + w, so the four
// heads sharing a KV head share every tile.  Split s covers keys
// [s*chunk, min(seq, (s+1)*chunk)), chunk = ceil(seq / ATTN_SPLITS).
// The block's four query vectors (2 KB) and its key tiles reach LDS by
// direct loads; two tile stages, so tile t + 1 is in flight while tile t is
// used.  Per tile of AT_T keys: lanes 2k and 2k+1 score key k over the even
// and odd 16-byte chunks of the row (joined by one DPP step), the online
// softmax update takes its maximum and sum by DPP steps, then lane l
// accumulates P.V for dims 2l, 2l+1 with each key's weight read out of its
// lane.  Launch with KvRing<KVT>::LDS bytes of dynamic LDS.
template <typename KVT>
__global__ __launch_bounds__(256) void attn_partial_kernel(const int *pos, const void *kc, const void *vc,
                                                           const float *q, unsigned long long *ts,
                                                           AttnArgs args) {
  ts_begin(ts);
  using G = KvRing<KVT>;
  extern __shared__ __attribute__((aligned(1024))) unsigned char attn_smem[];
  unsigned char *qs = attn_smem;           // [4][HD] f32
  unsigned char *ring = attn_smem + 2048;  // G::STAGES x (K tile | V tile)
  const int split = blockIdx.x / NKV, kvh = blockIdx.x % NKV;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int h = kvh * (NH / NKV) + wave;
  // the four query heads first in the load queue: every tile wait covers them
  if (wave < 2) lds_dma16(q + (size_t)kvh * (NH / NKV) * HD + wave * 256 + lane * 4, qs + wave * 1024);
  const int seq = *pos + 1;
  const int chunk = attn_chunk(seq);
  const int p0 = min(seq, split * chunk), p1 = min(seq, p0 + chunk);
  const KVT *Kb = (const KVT *)kc + (size_t)kvh * args.max_seq * HD;
  const KVT *Vb = (const KVT *)vc + (size_t)kvh * args.max_seq * HD;
  const int nt = (p1 - p0 + AT_T - 1) / AT_T;

  // tile t into stage t % STAGES: load i of wave w fills LDS block 4 i + w,
  // i.e. rows RPB (4 i + w) + lane / CPR, position lane % CPR; rows past the
  // split's end re-read its last row
  auto issue = [&](int t) {
    const int pb = p0 + t * AT_T, n = min(AT_T, p1 - pb);
    unsigned char *st = ring + (t % G::STAGES) * 2 * G::TB;
#pragma unroll
    for (int i = 0; i < G::BPT / 4; i++) {
      const int b = 4 * i + wave;
      const int row = b * G::RPB + lane / G::CPR;
      const int c = (lane % G::CPR) ^ kv_sw(row);
      const size_t g = (size_t)(pb + min(row, n - 1)) * HD + c * G::EPC;
      lds_dma16(Kb + g, st + b * 1024);
      lds_dma16(Vb + g, st + G::TB + b * 1024);
    }
  };
#pragma unroll
  for (int t = 0; t < G::STAGES; t++)
    if (t < nt) issue(t);

  const float scale = 1.0f / sqrtf((float)HD);
  const int key = lane >> 1, half = lane & 1;
  const float *qh = (const float *)qs + wave * HD;
  float m = -INFINITY, l = 0.f, o0 = 0.f, o1 = 0.f;
  for (int t = 0; t < nt; t++) {
    const int n = min(AT_T, p1 - p0 - t * AT_T);
    // this wave's loads of tile t are in (a later tile's may still fly),
    // then every wave's
    if (t + 1 < nt) __builtin_amdgcn_s_waitcnt(attn_vmcnt(G::LPW));
    else __builtin_amdgcn_s_waitcnt(attn_vmcnt(0));
    attn_barrier();
    const unsigned char *Kt = ring + (t % G::STAGES) * 2 * G::TB, *Vt = Kt + G::TB;
    const unsigned char *kr = Kt + key * G::RB;
    const int sw = kv_sw(key);
    float d0 = 0.f, d1 = 0.f;
#pragma unroll
    for (int i = 0; i < G::CPR / 2; i += 2) {
      const int c0 = 2 * i + half, c1 = c0 + 2;
      d0 = kdot((const KVT *)(kr + ((c0 ^ sw) << 4)), qh + c0 * G::EPC, d0);
      d1 = kdot((const KVT *)(kr + ((c1 ^ sw) << 4)), qh + c1 * G::EPC, d1);
    }
    float dot = d0 + d1;
    dot += dpp_mov<0xB1>(dot);  // quad_perm [1,0,3,2]: the pair's other half
    const bool valid = key < n;
    const float s = valid ? dot * scale : -INFINITY;
    const float mnew = fmaxf(m, wave_max_pairs(s));
    const float e = valid ? expf(s - mnew) : 0.f;
    const float corr = expf(m - mnew);
    l = l * corr + wave_sum_dpp(half ? 0.f : e);
    o0 *= corr;
    o1 *= corr;
    m = mnew;
    const int eb = __builtin_bit_cast(int, e);
#pragma unroll
    for (int j = 0; j < AT_T; j++) {
      const float ej = __builtin_bit_cast(float, __builtin_amdgcn_readlane(eb, 2 * j));  // 0 for j >= n
      const unsigned char *vr = Vt + j * G::RB;
      const int vc0 = sizeof(KVT) == 4 ? lane >> 1 : lane >> 2;
      const int vb = sizeof(KVT) == 4 ? (lane & 1) * 8 : (lane & 3) * 4;
      const float2 v = vpair((const KVT *)(vr + ((vc0 ^ kv_sw(j)) << 4) + vb));
      o0 = fmaf(ej, v.x, o0);
      o1 = fmaf(ej, v.y, o1);
    }
    if (t + G::STAGES < nt) {
      attn_barrier();  // every wave is done with this stage
      issue(t + G::STAGES);
    }
  }
  float *pp = args.part + ((size_t)h * ATTN_SPLITS + split) * (HD + 2);
  pp[lane * 2] = o0;
  pp[lane * 2 + 1] = o1;
  if (lane == 0) {
    pp[HD] = m;
    pp[HD + 1] = l;
  }
  ts_end(ts);
}

// Combine: one wave per query head; block b combines query head
// (NH / NKV) * (b % NKV) + b / NKV, on the XCD where its KV head's partials
// were written.  M = max m_s, L = sum l_s e^(m_s - M), o = sum o_s e^(m_s -
// M) / L (splits without keys carry m = -inf, l = 0).  Every load of the head
// (m, l of each split, both output dims of each split) is issued before the
// first is used: one memory round trip.
__global__ __launch_bounds__(64) void attn_combine_kernel(const float *part, float *out,
                                                          unsigned long long *ts) {
  ts_begin(ts);
  const int h = (NH / NKV) * ((int)blockIdx.x % NKV) + (int)blockIdx.x / NKV;
  const int lane = threadIdx.x;
  static_assert(ATTN_SPLITS <= 64, "one lane per split");
  const float *hp = part + (size_t)h * ATTN_SPLITS * (HD + 2);
  const float *mlp = hp + (lane & (ATTN_SPLITS - 1)) * (HD + 2) + HD;
  const bool lane_live = lane < ATTN_SPLITS;
  const float mv = lane_live ? mlp[0] : -INFINITY, lv = lane_live ? mlp[1] : 0.f;
  float2 o[ATTN_SPLITS];
#pragma unroll
  for (int s = 0; s < ATTN_SPLITS; s++) o[s] = *(const float2 *)(hp + s * (HD + 2) + lane * 2);
  // keep every load ahead of the first use (one memory round trip)
  __builtin_amdgcn_sched_barrier(0);
  const float M = wave_max_dpp(mv);
  const float wgt = lane_live ? expf(mv - M) : 0.f;
  const float L = wave_sum_dpp(lane_live ? lv * wgt : 0.f);
  float r0 = 0.f, r1 = 0.f;
#pragma unroll
  for (int s = 0; s < ATTN_SPLITS; s++) {
    const float ws = __shfl(wgt, s, 64);
    r0 = fmaf(ws, o[s].x, r0);
    r1 = fmaf(ws, o[s].y, r1);
  }
  out[h * HD + lane * 2] = r0 / L;
  out[h * HD + lane * 2 + 1] = r1 / L;
  ts_end(ts);
}

// ------------------------------------------------------- small kernels
// embeddingLookup: out[i] = table[token][i]
__global__ void embed_row_kernel(const uint16_t *table, int token, float *out) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < DIM) out[i] = h2f(table[(size_t)token * DIM + i]);
}

// The state a frame leaves (residual stream, normed, semantic logits), saved
// by the next frame's first kernel before it is overwritten; generate()
// puts it back when that next frame is discarded after an EOS.  Null x_prev:
// no save.
struct FrameSave {
  float *x_prev, *normed_prev, *logits_prev;
  const float *normed, *logits;
};

// multiCodebookEmbed: semantic row + 36 acoustic rows 8194 + k*23 + code_k,
// summed in that order.
__global__ void multi_codebook_kernel(const uint16_t *table, const uint32_t *sem,
                                      const uint32_t *codes, float *out, FrameSave sv) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= DIM) return;
  if (sv.x_prev) {
    sv.x_prev[i] = out[i];
    sv.normed_prev[i] = sv.normed[i];
    for (int j = i; j < SEMV; j += DIM) sv.logits_prev[j] = sv.logits[j];
  }
  // all 37 row indices, then all 37 row elements, then the ordered sum
  uint32_t row[NAC + 1];
  row[0] = sem[0];
#pragma unroll
  for (int k = 0; k < NAC; k++) row[k + 1] = 8194u + k * 23u + codes[k];
  uint16_t v[NAC + 1];
#pragma unroll
  for (int k = 0; k <= NAC; k++) v[k] = table[(size_t)row[k] * DIM + i];
  float s = 0.f;
#pragma unroll
  for (int k = 0; k <= NAC; k++) s += h2f(v[k]);
  out[i] = s;
}

// Final rmsNorm into `normed`; also advances the device decode position
// after every kernel of the step has read it.
__global__ __launch_bounds__(1024) void final_norm_kernel(const float *x, const uint16_t *w,
                                                          float eps, float *normed, int *pos,
                                                          unsigned long long *ts) {
  ts_begin(ts);
  __shared__ float red[16];
  const int tid = threadIdx.x;
  static_assert(DIM % 1024 == 0, "threads tile DIM");
  float xv[DIM / 1024], gv[DIM / 1024];
#pragma unroll
  for (int j = 0; j < DIM / 1024; j++) {  // the gains load with x, not after the reduction
    xv[j] = x[tid + j * 1024];
    gv[j] = h2f(w[tid + j * 1024]);
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < DIM / 1024; j++) s += xv[j] * xv[j];
  s = wave_sum_dpp(s);
  if ((tid & 63) == 0) red[tid >> 6] = s;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int k = 0; k < 16; k++) tot += red[k];
  const float rms = 1.0f / sqrtf(tot / (float)DIM + eps);
#pragma unroll
  for (int j = 0; j < DIM / 1024; j++) normed[tid + j * 1024] = xv[j] * rms * gv[j];
  if (pos != nullptr && tid == 0) *pos += 1;
  ts_end(ts);
}

// argmax with the reference's 256-lane strided scan and tree (strict '>').
// mask_valid > 0: indices 0 and >= mask_valid count as -inf (the host-side
// semantic masking of src/engine.ts:2556-2563).
// One block of 256 threads.
__device__ __forceinline__ void argmax_block(const float *x, int n, int mask_valid, uint32_t *result) {
  __shared__ float bv[256];
  __shared__ uint32_t bi[256];
  const int t = threadIdx.x;
  float best = -1e30f;
  uint32_t idx = 0;
  // thread t visits i = t, t+256, ... in order (strict >: the first maximum
  // wins), loading 16 elements per round trip
  constexpr int AB = 16;
  int i = t;
  for (; i + (AB - 1) * 256 < n; i += AB * 256) {
    float v[AB];
#pragma unroll
    for (int b = 0; b < AB; b++) v[b] = x[i + b * 256];
#pragma unroll
    for (int b = 0; b < AB; b++) {
      const int j = i + b * 256;
      const float w = mask_valid > 0 && (j == 0 || j >= mask_valid) ? -INFINITY : v[b];
      if (w > best) {
        best = w;
        idx = (uint32_t)j;
      }
    }
  }
  for (; i < n; i += 256) {
    float v = x[i];
    if (mask_valid > 0 && (i == 0 || i >= mask_valid)) v = -INFINITY;
    if (v > best) {
      best = v;
      idx = (uint32_t)i;
    }
  }
  bv[t] = best;
  bi[t] = idx;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (t < s && bv[t + s] > bv[t]) {
      bv[t] = bv[t + s];
      bi[t] = bi[t + s];
    }
    __syncthreads();
  }
  if (t == 0) result[0] = bi[0];
}
__global__ __launch_bounds__(256) void argmax_kernel(const float *x, int n, int mask_valid,
                                                     uint32_t *result) {
  argmax_block(x, n, mask_valid, result);
}

// ------------------------------------------------------------- generator
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
// Irwin-Hall(12) normal variate of (seed, stream, idx); bit-identical to
// the CPU generator (integer arithmetic, one exact conversion).
__device__ __forceinline__ float normal_variate(uint64_t seed, uint64_t stream, uint64_t idx) {
  const uint64_t s0 = mix64(seed) ^ stream;
  int64_t s = 0;
#pragma unroll
  for (uint64_t j = 0; j < 4; j++) {
    uint64_t h = mix64(s0 + (4 * idx + j + 1) * 0x9E3779B97F4A7C15ull);
    s += (int64_t)(h & 0xFFFFF) + (int64_t)((h >> 20) & 0xFFFFF) + (int64_t)((h >> 40) & 0xFFFFF);
  }
  return (float)(s - 6 * (int64_t)0xFFFFF) * 0x1p-20f;
}

// Box-Muller Gaussian of (seed, stream, idx), the FM noise (the reference's
// sqrt(-2 ln u1) cos(2 pi u2), src/engine.ts:1264-1273), bit-identical to the
// CPU generator: the same two hashed uniforms, and ln / cos by fixed
// sequences of correctly rounded double operations (series, no library
// transcendental):
//   u1 = N 2^-53, N = (h1 >> 11) + 1 = m 2^e, m in [sqrt(1/2), sqrt(2)):
//   ln u1 = (e - 53) ln 2 + 2 (s + s^3 p(s^2)), s = (m - 1) / (m + 1), p the
//   atanh series to s^14 / 17; u2 = U 2^-53: quadrant U >> 51, x = (U mod
//   2^51) 2^-51 pi / 2, cos x and sin x by Taylor series to x^20 / x^21.
__device__ __forceinline__ float fm_gauss(uint64_t seed, uint64_t stream, uint64_t idx) {
  constexpr double LOGC[8] = {0x1.5555555555555p-2, 0x1.999999999999ap-3, 0x1.2492492492492p-3,
                              0x1.c71c71c71c71cp-4, 0x1.745d1745d1746p-4, 0x1.3b13b13b13b14p-4,
                              0x1.1111111111111p-4, 0x1.e1e1e1e1e1e1ep-5};
  constexpr double COSC[10] = {-0x1.0000000000000p-1, 0x1.5555555555555p-5,  -0x1.6c16c16c16c17p-10,
                               0x1.a01a01a01a01ap-16, -0x1.27e4fb7789f5cp-22, 0x1.1eed8eff8d898p-29,
                               -0x1.93974a8c07c9dp-37, 0x1.ae7f3e733b81fp-45, -0x1.6827863b97d97p-53,
                               0x1.e542ba4020225p-62};
  constexpr double SINC[10] = {-0x1.5555555555555p-3, 0x1.1111111111111p-7,  -0x1.a01a01a01a01ap-13,
                               0x1.71de3a556c734p-19, -0x1.ae64567f544e4p-26, 0x1.6124613a86d09p-33,
                               -0x1.ae7f3e733b81fp-41, 0x1.952c77030ad4ap-49, -0x1.2f49b46814157p-57,
                               0x1.71b8ef6dcf572p-66};
  const uint64_t s0 = mix64(seed) ^ stream;
  const uint64_t h1 = mix64(s0 + (2 * idx + 1) * 0x9E3779B97F4A7C15ull);
  const uint64_t h2 = mix64(s0 + (2 * idx + 2) * 0x9E3779B97F4A7C15ull);
  const double d = (double)((h1 >> 11) + 1);  // exact
  const uint64_t bits = __builtin_bit_cast(uint64_t, d);
  int e = (int)((bits >> 52) & 0x7FF) - 1023;
  double m = __builtin_bit_cast(double, (bits & 0xFFFFFFFFFFFFFull) | 0x3FF0000000000000ull);
  if (m > 0x1.6a09e667f3bcdp+0) {
    m = __dmul_rn(m, 0.5);
    e += 1;
  }
  const double s = __ddiv_rn(__dsub_rn(m, 1.0), __dadd_rn(m, 1.0)), s2 = __dmul_rn(s, s);
  double p = LOGC[7];
#pragma unroll
  for (int k = 6; k >= 0; k--) p = __fma_rn(s2, p, LOGC[k]);
  const double lm = __dmul_rn(2.0, __fma_rn(__dmul_rn(s, s2), p, s));
  const double lu = __fma_rn((double)(e - 53), 0x1.62e42fefa39efp-1, lm);
  const double r = __dsqrt_rn(__dmul_rn(-2.0, lu));
  const uint64_t U = h2 >> 11;
  const int q = (int)(U >> 51);
  const double x = __dmul_rn(__dmul_rn((double)(U & ((1ull << 51) - 1)), 0x1p-51), 0x1.921fb54442d18p+0);
  const double x2 = __dmul_rn(x, x);
  double c = COSC[9], sn = SINC[9];
#pragma unroll
  for (int k = 8; k >= 0; k--) {
    c = __fma_rn(x2, c, COSC[k]);
    sn = __fma_rn(x2, sn, SINC[k]);
  }
  c = __fma_rn(x2, c, 1.0);
  sn = __fma_rn(__dmul_rn(x, x2), sn, x);
  const double cs = q == 0 ? c : q == 1 ? -sn : q == 2 ? -c : sn;
  return (float)__dmul_rn(r, cs);
}

__global__ void gen_f16_kernel(uint16_t *out, size_t n, uint64_t seed, uint64_t stream,
                               float mean, float std) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) {
    float t = __fmul_rn(normal_variate(seed, stream, i), std);
    out[i] = f2h_exact(__fadd_rn(mean, t));
  }
}

// KV rows for positions [0, npos): element (pos, c) of the reference layout
// [pos][1024] -> head-major cache [c/128][pos][c%128].  Values are the f16
// generator output (N(0,1) rounded to f16), held exactly in either cache type.
__device__ __forceinline__ float h2f_exact(uint16_t h) {  // subnormals kept
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 0x3ffu;
  if (e == 0) return __builtin_bit_cast(float, sign) + (sign ? -1.f : 1.f) * (float)m * 0x1p-24f;
  if (e == 31) return __builtin_bit_cast(float, sign | 0x7f800000u | (m << 13));
  return __builtin_bit_cast(float, sign | ((e + 112u) << 23) | (m << 13));
}
__device__ __forceinline__ void kv_put(float *p, uint16_t h) { *p = h2f_exact(h); }
__device__ __forceinline__ void kv_put(uint16_t *p, uint16_t h) { *p = h; }
template <typename KVT>
__global__ void gen_kv_kernel(KVT *cache, int max_seq, int npos, uint64_t seed, uint64_t stream) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t n = (size_t)npos * KVD;
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) {
    int p = (int)(i / KVD), c = (int)(i % KVD);
    kv_put(cache + ((size_t)(c >> 7) * max_seq + p) * HD + (c & 127),
           f2h_exact(normal_variate(seed, stream, i)));
  }
}

// --------------------------------------------- batched GEMM on MFMA (FM)
// The flow-matching transformer applies every weight to FMV = 6 vectors (3
// sequence positions x conditional/unconditional), so its GEMVs are thin
// GEMMs, out[v][row] = sum_k W[row][k] * y[v][k], run on
// v_mfma_f32_16x16x32_f16:
//  - A operand: the weights in tiles of FTR = 12 rows (every FM matrix has a
//    multiple of 256 x 12 rows, so each of the 256 CUs gets the same number
//    of tiles; 16-row tiles left 64 CUs idle on the 3072-row matrices),
//    pre-arranged once as [row tile][k chunk][48][8]: entry g*12 + m holds
//    row t*12 + m, k = chunk*32 + g*8 + e.  Lane l feeds MFMA row l%16 and k
//    group l/16; lanes of rows 12-15 load nothing (zeros), so one chunk's
//    operand is a contiguous 768-byte read;
//  - B operand: the packed input [k/8][BCOL] of 8-half groups, column v the
//    hi part f16(y_v) and column FMV+v the lo part f16(y_v - hi) (split2): W
//    is exactly f16, so D[.][v] + D[.][FMV+v] is the f32 dot product up to
//    rounding of order 2^-21 (f16 subnormals are kept by the conversion).
//    (The fused input kernel rounds hi to nearest, from the product y*g, and
//    lo from that same hi: order 2^-22.)  Columns 12-15
//    and rows 12-15 of D are never read.
// The kernel that produces a GEMM's input writes this packed form in its
// epilogue, with the next RMSNorm's gains already applied; the RMS scale
// itself multiplies the GEMM result (W.(x*g*r) = r * W.(x*g)), from
// per-tile sums of squares the producer also writes.
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
constexpr int FMV = 6;
constexpr int BCOL = 2 * FMV;
constexpr int FTR = 12;       // rows per FM weight tile
constexpr int SSQ_MAX = 256;  // partial sums of squares per vector (row tiles of a DIM output)

__device__ __forceinline__ void bpack_put(h8 *B, int v, int k, float y) {
  const _Float16 hi = (_Float16)y, lo = (_Float16)(y - (float)hi);  // one scalar conversion
  _Float16 *p = (_Float16 *)(B + (k >> 3) * BCOL);
  p[v * 8 + (k & 7)] = hi;
  p[(FMV + v) * 8 + (k & 7)] = lo;
}
// two consecutive k (k even) of vector v
__device__ __forceinline__ void bpack_put2(h8 *B, int v, int k, float y0, float y1) {
  h2 hi, lo;
  split2(y0, y1, hi, lo);
  _Float16 *p = (_Float16 *)(B + (k >> 3) * BCOL);
  *(h2 *)(p + v * 8 + (k & 7)) = hi;
  *(h2 *)(p + (FMV + v) * 8 + (k & 7)) = lo;
}
// four consecutive k (k % 4 == 0) of vector v
__device__ __forceinline__ void bpack_put4(h8 *B, int v, int k, f32x4 y) {
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  h4 hi, lo;
  const float x[4] = {y[0], y[1], y[2], y[3]};
  split_n<4>(x, hi, lo);
  _Float16 *p = (_Float16 *)(B + (k >> 3) * BCOL);
  *(h4 *)(p + v * 8 + (k & 7)) = hi;
  *(h4 *)(p + (FMV + v) * 8 + (k & 7)) = lo;
}

// W [M][K] row-major -> [M/12][K/32][48][8] (see above); M % 12 == 0
__global__ void pack_mfma_a_kernel(const uint16_t *W, uint16_t *Wp, int M, int K) {
  const size_t total = (size_t)M * K / 8;
  const int nch = K / 32;
  for (size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x; q < total;
       q += (size_t)gridDim.x * blockDim.x) {
    const int e = (int)(q % (4 * FTR));
    const size_t tc = q / (4 * FTR);
    const int c = (int)(tc % nch);
    const size_t tile = tc / nch;
    const int g = e / FTR, m = e - g * FTR;
    const uint16_t *src = W + (tile * FTR + m) * K + c * 32 + g * 8;
    *(u32x4 *)(Wp + q * 8) = *(const u32x4 *)src;
  }
}

struct Gemm6Args {
  const uint16_t *W, *W2;  // packed A (EPI_SWIGLU: W gate, W2 up)
  const h8 *B;             // packed input [K/8][BCOL]
  const float *ssq;        // RMSNorm of the input: nssq partial sums of squares per
  int nssq;                //   vector, ssq[p*FMV + v]; null: no norm
  float eps;
  float *out;              // outputs, vector stride os
  int os;
  float *out_k, *out_v;    // EPI_QKV
  h8 *Bn;                  // optional: next GEMM's packed input from the new values
  const uint16_t *gn;      //   times these gains (null: none)
  float *ssq_out;          //   and their sums of squares, vector-major [FMV][SSQ_MAX]
  // optional (EPI_RESID, the FM's last layer): this tile's share of the
  // acoustic projection of position 0 of each CFG branch (vectors 0 and 3),
  // ac_part[(b * NAC + o) * SSQ_MAX + tile] = sum over the tile's rows r of
  // acw[o][r] * acg[r] * y_b[r], and ac_ssq[b * SSQ_MAX + tile] = sum y_b[r]^2
  const uint16_t *acw, *acg;
  float *ac_part, *ac_ssq;
};

// Block = RG row tiles x KS k-slices (one wave each); a wave streams its
// tile's chunks (EPI_SWIGLU: the gate and up tiles), P chunks in flight, and
// k-slices are summed through LDS.  Grid = rows / (FTR RG).  KEEP: plain
// weight loads (cached in L2) instead of non-temporal ones.
template <int EPI, int K, int RG, int KS, int P, bool KEEP = false>
__global__ __launch_bounds__(RG * KS * 64) void gemm6_kernel(const uint16_t *W, const uint16_t *W2, const h8 *B,
                                                            const float *ssq, float *out, Gemm6Args args) {
  // the operands of the first loads arrive preloaded in SGPRs
  Gemm6Args a = args;
  a.W = W;
  a.W2 = W2;
  a.B = B;
  a.ssq = ssq;
  a.out = out;
  constexpr int TL = EPI == EPI_SWIGLU ? 2 : 1;
  constexpr int NC = K / 32, NCW = NC / KS;
  static_assert(NC % KS == 0 && NCW % P == 0, "shape");
  __shared__ f32x4 part[KS > 1 ? (KS - 1) * RG * TL : 1][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rg = wave / KS, kp = wave % KS;
  const int tile = blockIdx.x * RG + rg, row0 = tile * FTR, n = lane & 15;
  // A-operand lanes of rows 12-15 re-read rows 8-11 (the same cache lines,
  // so no extra traffic): rows of D depend only on the same rows of A, and
  // D rows 12-15 (lanes >= 48) are dropped.  The loads stay unconditional,
  // so the compiler issues them back to back.
  const bool drow = (lane >> 4) < FTR / 4;
  const uint16_t *wp[TL];
#pragma unroll
  for (int t = 0; t < TL; t++)
    wp[t] = (t ? a.W2 : a.W) +
            ((size_t)tile * NC * (4 * FTR) + (lane >> 4) * FTR + (n < FTR ? n : n - 4)) * 8;
  // lanes of columns 12-15 read a duplicate column (their D columns are unused)
  const h8 *bp = a.B + (lane >> 4) * BCOL + (n < BCOL ? n : n - FMV);
  // RMS scale of each input vector from the producer's partial sums
  // (nssq <= SSQ_MAX per vector, vector-major): one contiguous 16-byte load
  // per vector and lane, issued before the weights, whose loads return after
  // them.  Entries past nssq are masked (the buffer is shared by producers
  // of different partial counts).
  f32x4 sv[FMV];
  const bool norm = a.ssq != nullptr && kp == 0;  // wave-uniform
  if (norm) {
#pragma unroll
    for (int v = 0; v < FMV; v++) sv[v] = *(const f32x4 *)(a.ssq + v * SSQ_MAX + lane * 4);
  }
  // The epilogue's own operands (EPI_RESID: the residual values; the next
  // GEMM's norm gains) are loaded here too, so the wave that finishes the
  // block waits on no memory after its last MFMA.  Lanes of the dropped D
  // rows 12-15 read the tile's first rows instead.
  const int ev = n < FMV ? n : 0, er = row0 + (drow ? 4 * (lane >> 4) : 0);
  f32x4 eres = f32x4{0.f, 0.f, 0.f, 0.f};
  uint2 egn = uint2{0u, 0u};
  if (kp == 0) {
    if (EPI == EPI_RESID) eres = *(const f32x4 *)(a.out + (size_t)ev * a.os + er);
    if (a.Bn && a.gn) egn = *(const uint2 *)(a.gn + er);
  }
  // the acoustic-projection epilogue's weights and gains (below): lane
  // handles outputs idx = lane and lane + 64 < 2 NAC, each a 12-row slice
  uint2 acwv[2][FTR / 4], acgv[FTR / 4];
  if (EPI == EPI_RESID && a.ac_part && kp == 0) {
#pragma unroll
    for (int q = 0; q < FTR / 4; q++) acgv[q] = ((const uint2 *)(a.acg + row0))[q];
#pragma unroll
    for (int rep = 0; rep < 2; rep++) {
      const int o = (lane + 64 * rep) % NAC;
#pragma unroll
      for (int q = 0; q < FTR / 4; q++) acwv[rep][q] = ((const uint2 *)(a.acw + (size_t)o * DIM + row0))[q];
    }
  }
  u32x4 wb[P][TL];
  h8 bb[P];
  auto load = [&](int i, int d) {
    const int c = kp * NCW + i;
    bb[d] = bp[c * 4 * BCOL];
#pragma unroll
    for (int t = 0; t < TL; t++)
      wb[d][t] = KEEP ? *(const u32x4 *)(wp[t] + (size_t)c * (4 * FTR * 8))
                      : ldw(wp[t] + (size_t)c * (4 * FTR * 8));
  };
#pragma unroll
  for (int d = 0; d < P; d++) load(d, d);
  float rs[FMV];
#pragma unroll
  for (int v = 0; v < FMV; v++) rs[v] = 1.0f;
  if (norm) {
#pragma unroll
    for (int v = 0; v < FMV; v++) {
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < 4; j++) s += lane * 4 + j < a.nssq ? sv[v][j] : 0.f;
      rs[v] = 1.0f / sqrtf(wave_sum_dpp(s) / (float)DIM + a.eps);
    }
  }
  f32x4 acc[TL];
#pragma unroll
  for (int t = 0; t < TL; t++) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int c0 = 0; c0 < NCW; c0 += P) {
#pragma unroll
    for (int d = 0; d < P; d++) {
#pragma unroll
      for (int t = 0; t < TL; t++)
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, wb[d][t]), bb[d],
                                                        acc[t], 0, 0, 0);
      if (c0 + d + P < NCW) load(c0 + d + P, d);
    }
  }
  if (KS > 1) {
    if (kp > 0)
#pragma unroll
      for (int t = 0; t < TL; t++) part[((kp - 1) * RG + rg) * TL + t][lane] = acc[t];
    __syncthreads();
    if (kp > 0) return;
#pragma unroll
    for (int q = 1; q < KS; q++)
#pragma unroll
      for (int t = 0; t < TL; t++) acc[t] += part[((q - 1) * RG + rg) * TL + t][lane];
  }
  // hi + lo columns: lanes n < FMV then hold rows r..r+3 of vector v = n
#pragma unroll
  for (int t = 0; t < TL; t++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[t][j] += __shfl(acc[t][j], lane + FMV, 64);
  const int v = ev, r = row0 + 4 * (lane >> 4);
  float rv = rs[0];
#pragma unroll
  for (int u = 1; u < FMV; u++) rv = v == u ? rs[u] : rv;
  f32x4 y = acc[0] * rv;  // new values of rows r..r+3 (EPI_RESID: after the add)
  const bool live = n < FMV && drow;
  if (live) {
    if (EPI == EPI_SWIGLU) {
      const f32x4 u = acc[TL - 1] * rv;
#pragma unroll
      for (int j = 0; j < 4; j++) y[j] = (y[j] / (1.0f + expf(-y[j]))) * u[j];
      *(f32x4 *)(a.out + (size_t)v * a.os + r) = y;
    } else if (EPI == EPI_RESID) {
      y = y + eres;
      *(f32x4 *)(a.out + (size_t)v * a.os + r) = y;
    } else if (EPI == EPI_QKV) {
      if (r < QD)
        *(f32x4 *)(a.out + (size_t)v * QD + r) = y;
      else if (r < QD + KVD)
        *(f32x4 *)(a.out_k + (size_t)v * KVD + r - QD) = y;
      else
        *(f32x4 *)(a.out_v + (size_t)v * KVD + r - QD - KVD) = y;
    } else {
      *(f32x4 *)(a.out + (size_t)v * a.os + r) = y;
    }
  }
  if (a.Bn) {  // producer side of the next GEMM
    float s2 = live ? y[0] * y[0] + y[1] * y[1] + y[2] * y[2] + y[3] * y[3] : 0.f;
    s2 += __shfl_xor(s2, 16, 64);
    s2 += __shfl_xor(s2, 32, 64);
    if (live) {
      f32x4 z = y;
      if (a.gn) {
        const h2 g01 = __builtin_bit_cast(h2, egn.x), g23 = __builtin_bit_cast(h2, egn.y);
        z[0] *= (float)g01.x;
        z[1] *= (float)g01.y;
        z[2] *= (float)g23.x;
        z[3] *= (float)g23.y;
      }
      bpack_put4(a.Bn, v, r, z);
      if (a.ssq_out && lane < 16) a.ssq_out[v * SSQ_MAX + tile] = s2;
    }
  }
  if (EPI == EPI_RESID && a.ac_part) {
    // rows row0 .. row0 + FTR of vectors 0 and 3 through LDS, then lane
    // (b, o) = (idx / NAC, idx % NAC), idx = lane and lane + 64, sums its row
    // of the tile
    __shared__ __attribute__((aligned(16))) float acy[RG][2][FTR];
    if (live && (v == 0 || v == 3)) *(f32x4 *)&acy[rg][v / 3][4 * (lane >> 4)] = y;
    __builtin_amdgcn_s_waitcnt(0xC07F);  // the LDS writes of this wave are done
    float gv[FTR];
#pragma unroll
    for (int q = 0; q < FTR / 4; q++) {
      const uint2 gg = acgv[q];
      const h2 g01 = __builtin_bit_cast(h2, gg.x), g23 = __builtin_bit_cast(h2, gg.y);
      gv[4 * q] = (float)g01.x;
      gv[4 * q + 1] = (float)g01.y;
      gv[4 * q + 2] = (float)g23.x;
      gv[4 * q + 3] = (float)g23.y;
    }
#pragma unroll
    for (int rep = 0; rep < 2; rep++) {
      const int idx = lane + 64 * rep;
      if (idx < 2 * NAC) {
        const int b = idx / NAC;
        float sum = 0.f;
#pragma unroll
        for (int q = 0; q < FTR / 4; q++) {
          const uint2 ww = acwv[rep][q];
          const h2 w01 = __builtin_bit_cast(h2, ww.x), w23 = __builtin_bit_cast(h2, ww.y);
          sum = fmaf((float)w01.x * gv[4 * q], acy[rg][b][4 * q], sum);
          sum = fmaf((float)w01.y * gv[4 * q + 1], acy[rg][b][4 * q + 1], sum);
          sum = fmaf((float)w23.x * gv[4 * q + 2], acy[rg][b][4 * q + 2], sum);
          sum = fmaf((float)w23.y * gv[4 * q + 3], acy[rg][b][4 * q + 3], sum);
        }
        a.ac_part[(size_t)idx * SSQ_MAX + tile] = sum;
      }
    }
    if (lane < 2) {
      float s2 = 0.f;
#pragma unroll
      for (int r = 0; r < FTR; r++) s2 = fmaf(acy[rg][lane][r], acy[rg][lane][r], s2);
      a.ac_ssq[lane * SSQ_MAX + tile] = s2;
    }
  }
}

// ------------------------------------------------- top-p sampling (device)
// sampleTopP (src/engine.ts:247-289) over the semantic logits, with the
// generate() masking (index 0 and indices >= valid set to -inf,
// src/engine.ts:2556-2563):
//   s_i = f32(l_i / T); p_i = f32(exp(s_i - max)); q_i = f32(p_i / sum p)
//   with sum p in f64 (JS numbers), reduced in a fixed tree order;
//   order by q descending, equal q by ascending index (the reference's
//   stable sort);
//   cutoff = first rank whose running sum reaches top_p;
//   r = u * (sum of the first cutoff q); pick the first rank whose running
//   sum reaches r.
// No sort is needed.  Entry i has the unique 45-bit key
// (0x7FFFFFFF - bits(q_i)) << 14 | i, whose ascending order is the order
// above, and the exact mass floor(q_i * 2^62).  The running sums are exact
// integer sums, so "the first rank whose running sum reaches t" is the
// smallest key K with mass(keys <= K) >= t, found by a radix select (four
// passes over 12 + 11 + 11 + 11 key bits: per-bin masses and counts by LDS
// atomics, order-independent because they are integers; the first non-empty
// bin whose cumulative mass reaches t).  One select gives the cutoff key
// and its prefix mass resum; a second, with t = ceil(u * resum), gives the
// pick.  The reference's running sums round in f64, these are exact (to
// 2^-62 per entry): the picks differ only where a running sum lies within
// f64 rounding of a threshold.  u = (z >> 11) * 2^-53 for z the next output
// of a splitmix64 stream whose state lives at *rng (advanced once per
// call).  One block of TP_NT threads.
constexpr int TP_NT = 1024, TP_WAVES = TP_NT / 64;
constexpr int TP_MAXN = 9216;    // largest n
constexpr int TP_BINS = 4096;    // bins of the widest digit
static_assert(SEMV <= TP_MAXN && TP_MAXN <= 16384 && TP_BINS == 4 * TP_NT, "top-p sizes");

__device__ __forceinline__ uint64_t tp_mass(uint64_t key) {
  const float q = __builtin_bit_cast(float, 0x7FFFFFFFu - (uint32_t)(key >> 14));
  return (uint64_t)((double)q * 0x1p62);
}

// pub (or null): the frame's host-visible code slots [2][1 + NAC] (pinned
// host memory); the code also goes to slot (*frame - 1) & 1, the slot
// fm_finish_kernel filled for this frame before it advanced *frame.
__global__ __launch_bounds__(TP_NT) void topp_sample_kernel(const float *logits, int n, int valid,
                                                            const double *params, uint64_t *rng,
                                                            uint32_t *out, const int *frame, uint32_t *pub) {
  const double top_p = params[0], temp = params[1];  // in device memory: graphs stay valid
  __shared__ uint64_t key[TP_MAXN];       // first holds s_i, then p_i, as floats
  __shared__ uint64_t bmass[TP_BINS];     // also the f64 tree of the p sum
  __shared__ uint32_t bcnt[TP_BINS];
  __shared__ uint64_t wsum[TP_WAVES];
  __shared__ double red[TP_WAVES];
  __shared__ uint64_t sel_base, sel_incl, sel_key, target;
  __shared__ int sel;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float *sv = reinterpret_cast<float *>(key);
  // s_i and the max
  double mx = -INFINITY;
  for (int i = tid; i < n; i += TP_NT) {
    const float si = (i > 0 && i < valid) ? (float)((double)logits[i] / temp) : -INFINITY;
    sv[i] = si;
    mx = fmax(mx, (double)si);
  }
  for (int o = 32; o > 0; o >>= 1) mx = fmax(mx, __shfl_xor(mx, o, 64));
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = red[0];
  for (int w = 1; w < TP_WAVES; w++) mx = fmax(mx, red[w]);
  // p_i and their sum in f64: per thread, then a tree
  double *part = reinterpret_cast<double *>(bmass);
  double s = 0.0;
  for (int i = tid; i < n; i += TP_NT) {
    const float pi = (float)exp((double)sv[i] - mx);
    sv[i] = pi;
    s += (double)pi;
  }
  part[tid] = s;
  __syncthreads();
  for (int o = TP_NT / 2; o > 0; o >>= 1) {
    if (tid < o) part[tid] += part[tid + o];
    __syncthreads();
  }
  const double sum = part[0];
  // keys (each thread first reads its p_i: keys overwrite the floats)
  constexpr int PER = TP_MAXN / TP_NT;
  float pv[PER];
#pragma unroll
  for (int j = 0; j < PER; j++) {
    const int i = tid + j * TP_NT;
    pv[j] = i < n ? sv[i] : 0.f;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < PER; j++) {
    const int i = tid + j * TP_NT;
    if (i < n) {
      const float q = (float)((double)pv[j] / sum);
      key[i] = ((uint64_t)(0x7FFFFFFFu - __builtin_bit_cast(uint32_t, q)) << 14) | (uint32_t)i;
    }
  }
  // smallest key K with mass(keys <= K) >= t; returns K and that mass, or
  // found = false when the total mass stays below t
  auto select = [&](uint64_t t, uint64_t &kout, uint64_t &incl) -> bool {
    uint64_t prefix = 0, base = 0;
    for (int pass = 0; pass < 4; pass++) {
      const int width = pass == 0 ? 12 : 11, shift = 33 - 11 * pass;
      const int hi = shift + width, nb = 1 << width;
      for (int b = tid; b < TP_BINS; b += TP_NT) {
        bmass[b] = 0;
        bcnt[b] = 0;
      }
      if (tid == 0) sel = TP_BINS;
      __syncthreads();
      for (int i = tid; i < n; i += TP_NT) {
        const uint64_t k = key[i];
        if ((k >> hi) == prefix) {
          const int d = (int)((k >> shift) & (uint64_t)(nb - 1));
          atomicAdd((unsigned long long *)&bmass[d], (unsigned long long)tp_mass(k));
          atomicAdd(&bcnt[d], 1u);
        }
      }
      __syncthreads();
      // exclusive prefix of the mass of bins [0, 4 tid) over the block
      uint64_t m4 = 0;
#pragma unroll
      for (int j = 0; j < 4; j++) m4 += bmass[4 * tid + j];
      uint64_t incw = m4;
      for (int o = 1; o < 64; o <<= 1) {
        const uint64_t u = __shfl_up(incw, o, 64);
        if (lane >= o) incw += u;
      }
      if (lane == 63) wsum[wave] = incw;
      __syncthreads();
      uint64_t run = base + incw - m4;
      for (int w = 0; w < wave; w++) run += wsum[w];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int d = 4 * tid + j;
        if (d < nb && bcnt[d] > 0) {
          run += bmass[d];
          if (run >= t) {  // the running mass only grows: the smallest such d wins
            atomicMin(&sel, d);
            break;
          }
        }
      }
      __syncthreads();
      const int ds = sel;
      if (ds >= TP_BINS) return false;  // uniform: the total never reaches t
      // the owner of bin ds publishes the mass before it and including it
      if (tid == ds / 4) {
        uint64_t r2 = base + incw - m4;
        for (int w = 0; w < wave; w++) r2 += wsum[w];
        for (int d = 4 * tid; d < ds; d++)
          if (bcnt[d] > 0) r2 += bmass[d];
        sel_base = r2;
        sel_incl = r2 + bmass[ds];
      }
      __syncthreads();
      base = sel_base;
      prefix = (prefix << width) | (uint64_t)ds;
      incl = sel_incl;
      if (bcnt[ds] == 1) {
        // one key carries this prefix: the later passes would select its
        // digits with the same inclusive mass, so it is the answer
        for (int i = tid; i < n; i += TP_NT)
          if ((key[i] >> shift) == prefix) sel_key = key[i];
        __syncthreads();
        kout = sel_key;
        __syncthreads();  // every thread has read sel_key
        return true;
      }
      __syncthreads();  // bins and sel are reset by the next pass
    }
    kout = prefix;
    return true;
  };
  // cutoff: t = ceil(top_p * 2^62)
  if (tid == 0) {
    const double x = top_p * 0x1p62;
    target = x <= 0.0 ? 0ull : x >= 0x1p64 ? ~0ull : (uint64_t)ceil(x);
  }
  __syncthreads();
  uint64_t kc = 0, resum = 0;  // cutoff key and the mass of keys up to it
  if (!select(target, kc, resum)) {
    // the cutoff is n: resum is the total mass (every entry)
    for (int b = tid; b < TP_BINS; b += TP_NT) bmass[b] = 0;
    __syncthreads();
    uint64_t m = 0;
    for (int i = tid; i < n; i += TP_NT) m += tp_mass(key[i]);
    atomicAdd((unsigned long long *)&bmass[0], (unsigned long long)m);
    __syncthreads();
    resum = bmass[0];
    __syncthreads();
  }
  // draw: t = ceil(u * resum) with u = u53 * 2^-53, exactly
  if (tid == 0) {
    uint64_t z = (*rng += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    const uint64_t u53 = z >> 11;
    uint64_t lo = u53 * resum, hi = __umul64hi(u53, resum);
    const uint64_t add = (1ull << 53) - 1;
    lo += add;
    hi += lo < add;
    target = (hi << 11) | (lo >> 53);
  }
  __syncthreads();
  uint64_t kp = 0, dummy = 0;
  if (!select(target, kp, dummy)) select(0, kp, dummy);  // (t <= resum: not reached)
  if (tid == 0) {
    *out = (uint32_t)(kp & 0x3FFF);
    if (pub) pub[((*frame - 1) & 1) * (1 + NAC)] = (uint32_t)(kp & 0x3FFF);
  }
}

// ------------------------------------------------------------- FM kernels
// timeEmbedding (src/shaders.ts:579-602) for t
__global__ void time_embed_kernel(float *out, float t) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  const int half = DIM / 2;
  if (i >= half) return;
  float freq = expf((float)-9.210340371976184 * (float)i / (float)half);
  float ang = t * freq;
  out[i] = cosf(ang);
  out[half + i] = sinf(ang);
}

// CFG combine + Euler update (src/shaders.ts:611-648) of one coordinate:
// v = alpha*v_c + (1-alpha)*v_u; x' = x + v*dt
__device__ __forceinline__ float cfg_euler(float x, float vc, float vu, float alpha, float dt) {
  float v = __fadd_rn(__fmul_rn(alpha, vc), __fmul_rn(1.0f - alpha, vu));
  return __fadd_rn(x, __fmul_rn(v, dt));
}

struct FmStepArgs {
  float *xh;          // x_t history [nfe][NAC]; row s is the input of step s
  float *vel;         // velocity history [nfe-1][2][NAC]: row s - 1 written here
  const float *ac_part, *ac_ssq;  // the last FM layer's acoustic-projection partials
  const uint16_t *w_in;  // input_projection [DIM][NAC]
  const float *tproj;    // time projection of step s [DIM]
  const float *llm;      // llm projection [DIM]
  float *seq;            // [2][3][DIM]
  int step;
  float alpha, dt;
  const float *noise;    // step 0: x_t = noise, or (null) the device generator's
  const uint64_t *noise_seed;  //   fm_gauss(seed, noise_stream, frame * NAC + i)
  uint64_t noise_stream;
  const int *frame;
  h8 *Bn;                // packed input of the first layer's QKV GEMM,
  const uint16_t *gn;    //   times its attention-norm gains,
  float *ssq_out;        //   and sums of squares, vector-major [FMV][SSQ_MAX]
  // step 0: a block past the grid's DIM / 256 takes the (masked) argmax of
  // the semantic logits (argmax_kernel's work, off the FM's critical path)
  const float *sem_logits;
  int sem_mask;
  uint32_t *sem_code;
};

// The velocities of an Euler step (acoustic_codebook_output(RMSNorm(position
// 0)) of both CFG branches, src/engine.ts:1210-1224) from the partial sums
// the last FM layer's down GEMM leaves per 12-row tile: vs[b * NAC + o] =
// rs_b * sum over tiles of ac_part, rs_b = 1 / sqrt(sum ac_ssq / DIM + eps).
// Block of 256 threads; every thread calls it; vs is valid after the
// barrier inside.
__device__ __forceinline__ void fm_velocity(const float *ac_part, const float *ac_ssq, float *vs) {
  static_assert(SSQ_MAX == 256 && DIM / FTR == SSQ_MAX, "one partial per tile, 4 per lane");
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  f32x4 q[2], p[(2 * NAC + 3) / 4];
#pragma unroll
  for (int b = 0; b < 2; b++) q[b] = *(const f32x4 *)(ac_ssq + b * SSQ_MAX + 4 * lane);
#pragma unroll
  for (int i = 0; i < (2 * NAC + 3) / 4; i++) {
    const int idx = w + 4 * i;
    p[i] = idx < 2 * NAC ? *(const f32x4 *)(ac_part + (size_t)idx * SSQ_MAX + 4 * lane) : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  float rs[2];
#pragma unroll
  for (int b = 0; b < 2; b++)
    rs[b] = 1.0f / sqrtf(wave_sum_dpp((q[b][0] + q[b][1]) + (q[b][2] + q[b][3])) / (float)DIM + 1e-5f);
#pragma unroll
  for (int i = 0; i < (2 * NAC + 3) / 4; i++) {
    const int idx = w + 4 * i;
    const float sum = wave_sum_dpp((p[i][0] + p[i][1]) + (p[i][2] + p[i][3]));
    if (idx < 2 * NAC && lane == 0) vs[idx] = sum * rs[idx / NAC];
  }
  __syncthreads();
}

// Start of Euler step s: x_s (from x_{s-1} and the CFG velocity of step
// s-1, or the noise at s=0), x_t_proj = input_projection(x_s), and both CFG
// sequences [x_t_proj, time_proj, llm | 0] (src/engine.ts:1292-1349).
__global__ __launch_bounds__(256) void fm_step_in_kernel(const uint16_t *w_in, const float *ac_part,
                                                         const float *ac_ssq, float *xh, FmStepArgs args) {
  // the first loads' pointers arrive preloaded in SGPRs
  FmStepArgs a = args;
  a.w_in = w_in;
  a.ac_part = ac_part;
  a.ac_ssq = ac_ssq;
  a.xh = xh;
  __shared__ float xs[NAC];
  __shared__ float vs[2 * NAC];
  const int t = threadIdx.x;
  if (blockIdx.x == DIM / 256) {  // launched with this block at step 0 only
    argmax_block(a.sem_logits, SEMV, a.sem_mask, a.sem_code);
    return;
  }
  const int row = blockIdx.x * 256 + t;  // grid covers DIM exactly
  // this row's input-projection weights, time/llm projections and gain do
  // not depend on x_s: issued first, they arrive while x_s is formed
  uint2 wr[NAC / 4];
#pragma unroll
  for (int j = 0; j < NAC / 4; j++) wr[j] = ((const uint2 *)(a.w_in + (size_t)row * NAC))[j];
  const float tp = a.tproj[row], lp = a.llm[row];
  const float g = h2f(a.gn[row]);
  // x_{s-1} too, so that no load waits behind the velocity's barrier
  const float xprev = a.step > 0 && t < NAC ? a.xh[(a.step - 1) * NAC + t] : 0.f;
  if (a.step > 0) {
    fm_velocity(a.ac_part, a.ac_ssq, vs);
    if (blockIdx.x == 0 && t < 2 * NAC) a.vel[(size_t)(a.step - 1) * 2 * NAC + t] = vs[t];
  }
  if (t < NAC) {
    float x;
    if (a.step == 0) {
      x = a.noise ? a.noise[t] : fm_gauss(*a.noise_seed, a.noise_stream, (uint64_t)(*a.frame) * NAC + t);
    } else {
      x = cfg_euler(xprev, vs[t], vs[NAC + t], a.alpha, a.dt);
    }
    xs[t] = x;
    if (blockIdx.x == 0) a.xh[a.step * NAC + t] = x;
  }
  __syncthreads();
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < NAC / 4; j++) {
    const h2 w01 = __builtin_bit_cast(h2, wr[j].x), w23 = __builtin_bit_cast(h2, wr[j].y);
    acc = fmaf((float)w01.x, xs[4 * j], acc);
    acc = fmaf((float)w01.y, xs[4 * j + 1], acc);
    acc = fmaf((float)w23.x, xs[4 * j + 2], acc);
    acc = fmaf((float)w23.y, xs[4 * j + 3], acc);
  }
  const float y[FMV] = {acc, tp, lp, acc, tp, 0.f};
  __shared__ float red[4][FMV];
#pragma unroll
  for (int v = 0; v < FMV; v++) {
    a.seq[v * DIM + row] = y[v];
    bpack_put(a.Bn, v, row, y[v] * g);
    const float s2 = wave_sum_dpp(y[v] * y[v]);
    if ((t & 63) == 0) red[t >> 6][v] = s2;
  }
  __syncthreads();
  if (t < FMV) a.ssq_out[t * SSQ_MAX + blockIdx.x] = red[0][t] + red[1][t] + red[2][t] + red[3][t];
}

// Bidirectional 3-token GQA attention of both CFG branches: grid (NH, 2),
// one wave per (head, branch); q [6][QD], k/v [6][KVD], out [6][QD], and
// out in the packed form of the O projection's input.
__global__ __launch_bounds__(64) void fm_attn_kernel(const float *q, const float *k,
                                                     const float *v, float *out, h8 *Bn) {
  const int h = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
  const int kvh = h / (NH / NKV);
  const float scale = 1.0f / sqrtf((float)HD);
  float qv[3][2], kv[3][2], vv[3][2];
#pragma unroll
  for (int i = 0; i < 3; i++) {
    const int vec = b * 3 + i;
    qv[i][0] = q[(size_t)vec * QD + h * HD + lane * 2];
    qv[i][1] = q[(size_t)vec * QD + h * HD + lane * 2 + 1];
    kv[i][0] = k[(size_t)vec * KVD + kvh * HD + lane * 2];
    kv[i][1] = k[(size_t)vec * KVD + kvh * HD + lane * 2 + 1];
    vv[i][0] = v[(size_t)vec * KVD + kvh * HD + lane * 2];
    vv[i][1] = v[(size_t)vec * KVD + kvh * HD + lane * 2 + 1];
  }
#pragma unroll
  for (int i = 0; i < 3; i++) {
    float s[3];
#pragma unroll
    for (int j = 0; j < 3; j++) s[j] = wave_sum_dpp(qv[i][0] * kv[j][0] + qv[i][1] * kv[j][1]) * scale;
    float mx = fmaxf(fmaxf(s[0], s[1]), s[2]);
    float e0 = expf(s[0] - mx), e1 = expf(s[1] - mx), e2 = expf(s[2] - mx);
    float sum = e0 + e1 + e2;
    e0 /= sum; e1 /= sum; e2 /= sum;
    const int vec = b * 3 + i;
    const float o0 = e0 * vv[0][0] + e1 * vv[1][0] + e2 * vv[2][0];
    const float o1 = e0 * vv[0][1] + e1 * vv[1][1] + e2 * vv[2][1];
    out[(size_t)vec * QD + h * HD + lane * 2] = o0;
    out[(size_t)vec * QD + h * HD + lane * 2 + 1] = o1;
    bpack_put2(Bn, vec, h * HD + lane * 2, o0, o1);
  }
}

// End of the Euler loop: last CFG/Euler update, then fsqQuantize (round
// half to even) into the device acoustic codes; also advances the frame
// counter of the noise generator.  pub (or null): host-visible code slots
// [2][1 + NAC] in pinned host memory; the frame's acoustic codes and the
// device semantic code go to slot frame & 1 (a later kernel may replace
// the semantic code), so the host reads a frame's codes without a copy.
__global__ __launch_bounds__(256) void fm_finish_kernel(float *xh, float *vel, const float *ac_part,
                                                       const float *ac_ssq, int last, float alpha, float dt,
                                                       uint32_t *codes, int levels, int *frame_counter,
                                                       const uint32_t *sem_code, uint32_t *pub) {
  __shared__ float vs[2 * NAC];
  const int t = threadIdx.x;
  const float xprev = t < NAC ? xh[last * NAC + t] : 0.f;  // issued before the velocity's barrier
  // read before the barrier inside fm_velocity; thread 0 advances it after
  const int fc = frame_counter ? *frame_counter : 0;
  uint32_t *slot = pub ? pub + (fc & 1) * (1 + NAC) : nullptr;
  fm_velocity(ac_part, ac_ssq, vs);
  if (t < 2 * NAC) vel[(size_t)last * 2 * NAC + t] = vs[t];
  if (t < NAC) {
    float x = cfg_euler(xprev, vs[t], vs[NAC + t], alpha, dt);
    xh[(last + 1) * NAC + t] = x;
    float c = fminf(fmaxf(x, -1.0f), 1.0f);
    float top = (float)(levels - 1);
    float sc = rintf((c + 1.0f) * 0.5f * top);
    const uint32_t code = (uint32_t)fminf(fmaxf(sc, 0.0f), top) + 2u;
    codes[t] = code;
    if (slot) slot[1 + t] = code;
  }
  if (slot && t == NAC) slot[0] = *sem_code;
  if (t == 0 && frame_counter) *frame_counter += 1;
}


}  // namespace vx
