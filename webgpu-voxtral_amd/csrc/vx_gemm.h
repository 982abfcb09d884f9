// vx_gemm.h -- the prefill's projections as hand-written gfx950 MFMA GEMMs:
//   C[s][col][m] = sum_{k in slice s} W[m][k] * (Bhi[col][k] + Blo[col][k])
// W: f16 weights, row-major M x K as loaded (the decode GEMVs read the same
// copy).  B: 2 nt rows of K halves, the hi half of each activation column in
// row col and its f16 residual (lo) in row nt + col, as the prefill's
// producer kernels write them.  Hi and lo go through the same MFMA
// accumulator, so the product keeps f32 accuracy.  The K range is split
// into S_out slices whose partial sums land in S_out consecutive [nt][M]
// blocks of C; the consumer adds them (fixed order, so results are
// deterministic).
//
// Tile: 256 weight rows x 64 columns (128 B rows: 64 hi + 64 lo) per block
// of 4 waves; wave w owns weight rows 64 w .. + 64 and all 128 B rows, as
// 2 x 2 tiles of v_mfma_f32_32x32x16_f16 (hi and lo accumulate into the
// same tile).  A k-tile is 64 halves: 256 + 128 rows of 128 B = 48 KB of
// LDS, filled by direct global->LDS loads (global_load_lds_dwordx4, 1 KB per
// instruction = 8 rows) into a ring of 3 stages (144 KB).  Per k-tile a wave
// issues 32 MFMAs, 24 ds_read_b128 and 12 direct loads; the schedule
// interleaves them (MFMA, read, load, MFMA, read ...) so that neither the
// LDS reads nor the loads' issue stall the matrix pipe, reads of step q + 1
// run under the MFMAs of step q, and the stage barrier sits before the last
// step so the next stage's first fragments are read under it.
//
// Two grids:
//  - gemm_split_kernel: one tile per block, K split in KS = gridDim.y
//    slices (S_out = KS); for shapes with at most one block per CU.
//  - gemm_stream_kernel: one block per CU, each doing an equal share of the
//    column tile's (row tile, k-tile) sequence; S_out = the most blocks a
//    tile is split over (rounded up to 1, 2, 4 or 8); for shapes with more
//    tiles than CUs, which would otherwise run in uneven rounds.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>
#include <type_traits>

namespace vx {

typedef _Float16 gm_h8 __attribute__((ext_vector_type(8)));
typedef float gm_f32x4 __attribute__((ext_vector_type(4)));
typedef float gm_f32x16 __attribute__((ext_vector_type(16)));

constexpr int GM_BM = 256;                 // weight rows per tile
constexpr int GM_BN = 64;                  // activation columns per tile
constexpr int GM_BK = 64;                  // halves per k-tile
constexpr int GM_ROWB = 128;               // bytes per LDS row (one k-tile of one row)
constexpr int GM_STAGE = (GM_BM + 2 * GM_BN) * GM_ROWB;  // 48 KB
constexpr int GM_S = 3;                    // stages in the LDS ring
constexpr int GM_LDS = GM_S * GM_STAGE;    // 144 KB
constexpr int GM_LOADS = 12;               // direct loads per wave per k-tile

// s_waitcnt immediate for vmcnt(vm) with the other counters left open
constexpr int gm_vmcnt(int vm) { return (vm & 15) | ((vm >> 4) << 14) | (7 << 4) | (15 << 8); }
constexpr int GM_LGKM0 = 0xC07F;  // lgkmcnt(0)

// LDS position of 16-byte chunk c of stage row R: c ^ ((R >> 1) & 7), so the
// 32 rows one fragment read touches spread over the banks
__device__ __forceinline__ int gm_key(int row) { return (row >> 1) & 7; }

// The k-tile pipeline shared by both grids.  State: fragment registers,
// accumulators, per-lane LDS offsets; the caller supplies the source of each
// k-tile's loads.
struct GmLane {
  int lane, wave, r, h;
  int roff[6], rkey[6];  // LDS row offset and key of fragment f (A: f < 2, B: 2 + 2 hl + j)
  __device__ __forceinline__ GmLane(int tid) {
    lane = tid & 63;
    wave = tid >> 6;
    r = lane & 31;
    h = lane >> 5;
#pragma unroll
    for (int f = 0; f < 6; f++) {
      const int row = f < 2 ? wave * 64 + f * 32 + r : GM_BM + ((f - 2) >> 1) * GM_BN + ((f - 2) & 1) * 32 + r;
      roff[f] = row * GM_ROWB;
      rkey[f] = gm_key(row);
    }
  }
  // direct load i of this wave fills stage row 8 (4 i + w) + lane / 8
  // (i < 8: weight rows, else B rows), position lane % 8, which holds chunk
  // (lane % 8) ^ key(row)
  __device__ __forceinline__ int load_row(int i) const { return 8 * (4 * i + wave) + (lane >> 3); }
  __device__ __forceinline__ int load_chunk(int i) const { return (lane & 7) ^ gm_key(load_row(i)); }
};

__device__ __forceinline__ void gm_direct(const uint16_t *src, unsigned char *lds_row_block) {
  __builtin_amdgcn_global_load_lds((const void *)src, (__attribute__((address_space(3))) void *)lds_row_block, 16,
                                   0, 0);
}

__device__ __forceinline__ void gm_read(const GmLane &L, const unsigned char *stage, int q, gm_h8 (&fr)[6]) {
  const int c = 2 * q + L.h;
#pragma unroll
  for (int f = 0; f < 6; f++) fr[f] = *(const gm_h8 *)(stage + L.roff[f] + ((c ^ L.rkey[f]) << 4));
}

__device__ __forceinline__ void gm_mfma(gm_f32x16 (&acc)[2][2], const gm_h8 (&fr)[6]) {
#pragma unroll
  for (int hl = 0; hl < 2; hl++)
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int j = 0; j < 2; j++)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fr[i], fr[2 + 2 * hl + j], acc[i][j], 0, 0, 0);
}

// 8 MFMAs, 6 LDS reads, 3 direct loads: M R L M R  M R L M R  M R L M R  M M
__device__ __forceinline__ void gm_interleave() {
#pragma unroll
  for (int k = 0; k < 3; k++) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
  }
  __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
}

__device__ __forceinline__ void gm_zero(gm_f32x16 (&acc)[2][2]) {
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;
}

// acc[i][j][e] is weight row 64 w + 32 i + 8 (e / 4) + 4 h + e % 4 of the
// tile, column 32 j + r: written as C[col][m] with float4 stores
__device__ __forceinline__ void gm_store(const GmLane &L, const gm_f32x16 (&acc)[2][2], float *C, int ldc, int col0,
                                         int m0, bool zero) {
  float *cp = C + (size_t)(col0 + L.r) * ldc + m0 + L.wave * 64 + 4 * L.h;
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int g4 = 0; g4 < 4; g4++)
        *(gm_f32x4 *)(cp + (size_t)j * 32 * ldc + i * 32 + 8 * g4) =
            zero ? gm_f32x4{0.f, 0.f, 0.f, 0.f}
                 : gm_f32x4{acc[i][j][4 * g4], acc[i][j][4 * g4 + 1], acc[i][j][4 * g4 + 2], acc[i][j][4 * g4 + 3]};
}

// One k-tile iteration t of the pipeline.  Stage `stage` holds k-tile t,
// stage nxt k-tile t + 1 (in flight); f0 holds step 0's fragments.  The 12
// direct loads of the pending k-tile (the one the previous iteration's
// barrier freed a stage for) are finished in steps 0-2 (loads 3-11, unless
// FIRST: none pending yet), then after this iteration's barrier a new
// k-tile's loads 0-2 go out in step 3 (`next_src` switches the source).
// Each k-tile's 12 loads stay contiguous in issue order, so at the barrier
// k-tile t + 1 is in once at most 12 (S - 2) younger loads, plus `extra`
// stores issued since, are outstanding.
template <bool FIRST, typename Src, typename Next>
__device__ __forceinline__ void gm_iteration(const GmLane &L, unsigned char *smem, gm_f32x16 (&acc)[2][2],
                                             gm_h8 (&f0)[6], gm_h8 (&f1)[6], int &stage, int &pend_stage,
                                             int extra, const Src &src, const Next &next_src) {
  const int nxt = stage + 1 == GM_S ? 0 : stage + 1;
  const unsigned char *cur = smem + stage * GM_STAGE;
  // step q's reads with loads i0 .. i0 + 2 between them in program order
  // (the compiler keeps LDS reads and direct loads, which may alias, in
  // that order; the schedule then interleaves both with the MFMAs)
  auto read_load = [&](const unsigned char *rs, int q, gm_h8 (&fr)[6], int i0) {
    const int c = 2 * q + L.h;
    unsigned char *ls = smem + pend_stage * GM_STAGE;
#pragma unroll
    for (int k = 0; k < 3; k++) {
      fr[2 * k] = *(const gm_h8 *)(rs + L.roff[2 * k] + ((c ^ L.rkey[2 * k]) << 4));
      gm_direct(src(i0 + k), ls + (4 * (i0 + k) + L.wave) * 1024);
      fr[2 * k + 1] = *(const gm_h8 *)(rs + L.roff[2 * k + 1] + ((c ^ L.rkey[2 * k + 1]) << 4));
    }
  };
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (!FIRST) read_load(cur, 1, f1, 3);
  else gm_read(L, cur, 1, f1);
  gm_mfma(acc, f0);
  gm_interleave();
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (!FIRST) read_load(cur, 2, f0, 6);
  else gm_read(L, cur, 2, f0);
  gm_mfma(acc, f1);
  gm_interleave();
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (!FIRST) read_load(cur, 3, f1, 9);
  else gm_read(L, cur, 3, f1);
  gm_mfma(acc, f0);
  gm_interleave();
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(GM_LGKM0);
  if (extra == 0) __builtin_amdgcn_s_waitcnt(gm_vmcnt(12 * (GM_S - 2)));
  else if (extra == 16) __builtin_amdgcn_s_waitcnt(gm_vmcnt(12 * (GM_S - 2) + 16));
  else __builtin_amdgcn_s_waitcnt(gm_vmcnt(12 * (GM_S - 2) + 32));
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  // every wave is done with stage `stage`: it takes the new k-tile
  next_src();
  pend_stage = stage;
  read_load(smem + nxt * GM_STAGE, 0, f0, 0);
  gm_mfma(acc, f1);
  gm_interleave();
  __builtin_amdgcn_sched_barrier(0);
  stage = nxt;
}

// Split-K grid: block (x, s) computes tile x (XCD-grouped, m-major) over K
// slice s of KS = gridDim.y and writes C block s.  Needs M % 256 == 0,
// nt % 64 == 0, K % (64 KS) == 0.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void gemm_split_kernel(
    const uint16_t *__restrict__ W, int M, int K, const uint16_t *__restrict__ B, int nt, float *__restrict__ C,
    int ldc) {
  extern __shared__ __attribute__((aligned(16))) unsigned char gm_smem[];
  const GmLane L(threadIdx.x);
  const int n_tiles = nt / GM_BN, m_tiles = M / GM_BM;
  // tiles m-major; the blocks b with b % 8 == x take the x-th eighth.
  // Workgroups are dealt to the 8 XCDs round-robin (from a starting XCD that
  // varies between launches), so blocks with equal b % 8 share an XCD: the
  // column tiles sharing a weight tile run together and one L2 serves the
  // re-reads
  int mt, ntl;
  {
    const int b = blockIdx.x, tiles = m_tiles * n_tiles;
    const int tile = (tiles & 7) == 0 ? (b & 7) * (tiles >> 3) + (b >> 3) : b;
    mt = tile / n_tiles;
    ntl = tile - mt * n_tiles;
  }
  const int kh = K / gridDim.y, kb = blockIdx.y * kh, nk = kh / GM_BK, last = nk - 1;
  const uint16_t *base[GM_LOADS];
#pragma unroll
  for (int i = 0; i < GM_LOADS; i++) {
    const int row = L.load_row(i), chunk = L.load_chunk(i);
    if (i < 8) {
      base[i] = W + (size_t)(mt * GM_BM + row) * K + kb + chunk * 8;
    } else {
      const int br = row - GM_BM, hl = br / GM_BN, col = br % GM_BN;
      base[i] = B + (size_t)(hl * nt + ntl * GM_BN + col) * K + kb + chunk * 8;
    }
  }
  gm_f32x16 acc[2][2];
  gm_zero(acc);
  gm_h8 f0[6], f1[6];
  // prologue: k-tiles 0 .. S-1 fill the ring (indices past the last k-tile
  // reload it, so every iteration issues the same number of loads)
#pragma unroll
  for (int s = 0; s < GM_S; s++)
#pragma unroll
    for (int i = 0; i < GM_LOADS; i++)
      gm_direct(base[i] + min(s, last) * GM_BK, gm_smem + s * GM_STAGE + (4 * i + L.wave) * 1024);
  __builtin_amdgcn_s_waitcnt(gm_vmcnt(12 * (GM_S - 1)));
  __builtin_amdgcn_s_barrier();
  gm_read(L, gm_smem, 0, f0);
  int stage = 0, pend_stage = 0, pend_kt = min(GM_S, last);
  auto src = [&](int i) { return base[i] + pend_kt * GM_BK; };
  int t = 0;
  auto next = [&]() { pend_kt = min(t + GM_S, last); };
  gm_iteration<true>(L, gm_smem, acc, f0, f1, stage, pend_stage, 0, src, next);
  for (t = 1; t < nk; t++) gm_iteration<false>(L, gm_smem, acc, f0, f1, stage, pend_stage, 0, src, next);
  // the ring's last loads (re-reads) must land before this block's LDS is released
  __builtin_amdgcn_s_waitcnt(gm_vmcnt(0));
  gm_store(L, acc, C + (size_t)blockIdx.y * nt * ldc, ldc, ntl * GM_BN, mt * GM_BM, false);
}

// Balanced grid: G blocks (G / 8 a multiple of n_tiles).  Block lb works on
// column tile c = lb % n_tiles, share j = lb / n_tiles of that column's
// sequence g = mt * nk + kt, g in [j L, (j + 1) L).  A tile is split into
// the segments of the blocks whose shares overlap it; the segment of block j
// goes to C block j - j0(mt), j0(mt) = mt nk / L (its first block), and the
// block holding a tile's last segment writes zeros to the C blocks after it,
// up to the ns blocks the consumer reads.  The n_tiles blocks of a share
// read the same weight k-tiles at the same time; the blocks b with equal
// b % 8 (one XCD, as workgroups are dealt to the XCDs round-robin) hold
// whole shares, so one L2 serves them.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void gemm_stream_kernel(
    const uint16_t *__restrict__ W, int M, int K, const uint16_t *__restrict__ B, int nt, float *__restrict__ C,
    int ldc, int Lshare, int ns) {
  extern __shared__ __attribute__((aligned(16))) unsigned char gm_smem[];
  const GmLane L(threadIdx.x);
  const int n_tiles = nt / GM_BN, m_tiles = M / GM_BM, nk = K / GM_BK;
  const int G = gridDim.x;
  const int lb = (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3);
  const int c = lb % n_tiles, j = lb / n_tiles;
  const int total = m_tiles * nk;
  const int g0 = min(j * Lshare, total), g1 = min(g0 + Lshare, total);
  if (g0 >= g1) return;
  const int last = g1 - 1;
  const size_t slot_stride = (size_t)nt * ldc;
  // per-lane offsets of the direct loads from the k-tile's weight / B origin
  size_t off[GM_LOADS];
#pragma unroll
  for (int i = 0; i < GM_LOADS; i++) {
    const int row = L.load_row(i), chunk = L.load_chunk(i);
    if (i < 8) {
      off[i] = (size_t)row * K + chunk * 8;
    } else {
      const int br = row - GM_BM, hl = br / GM_BN, col = br % GM_BN;
      off[i] = (size_t)(hl * nt + c * GM_BN + col) * K + chunk * 8;
    }
  }
  gm_f32x16 acc[2][2];
  gm_zero(acc);
  // zeros for the C blocks past each tile whose last segment is this
  // block's (issued before the ring's first loads, so the stores are older
  // than every load the pipeline counts)
  for (int mt = g0 / nk; mt <= last / nk; mt++) {
    if ((mt + 1) * nk - 1 > last) break;  // the tile goes on in the next block
    for (int sl = j - mt * nk / Lshare + 1; sl < ns; sl++)
      gm_store(L, acc, C + sl * slot_stride, ldc, c * GM_BN, mt * GM_BM, true);
  }
  gm_h8 f0[6], f1[6];
#pragma unroll
  for (int s = 0; s < GM_S; s++) {
    const int g = min(g0 + s, last), mt = g / nk, kt = g - mt * nk;
    const uint16_t *wa = W + (size_t)mt * GM_BM * K + kt * GM_BK, *ba = B + kt * GM_BK;
#pragma unroll
    for (int i = 0; i < GM_LOADS; i++)
      gm_direct((i < 8 ? wa : ba) + off[i], gm_smem + s * GM_STAGE + (4 * i + L.wave) * 1024);
  }
  __builtin_amdgcn_s_waitcnt(gm_vmcnt(12 * (GM_S - 1)));
  __builtin_amdgcn_s_barrier();
  gm_read(L, gm_smem, 0, f0);
  // pending loads' position (iteration min(g + S, last)), advanced one k-tile
  // per iteration without divisions
  int p_mt, p_kt;
  {
    const int pg = min(g0 + GM_S, last);
    p_mt = pg / nk;
    p_kt = pg - p_mt * nk;
  }
  const uint16_t *wa = W + (size_t)p_mt * GM_BM * K + p_kt * GM_BK, *ba = B + p_kt * GM_BK;
  auto src = [&](int i) { return (i < 8 ? wa : ba) + off[i]; };
  int g = g0;
  bool first = true;
  auto next = [&]() {
    if (!first && g + GM_S <= last) {
      if (++p_kt == nk) {
        p_kt = 0;
        ++p_mt;
      }
      wa = W + (size_t)p_mt * GM_BM * K + p_kt * GM_BK;
      ba = B + p_kt * GM_BK;
    }
  };
  int stage = 0, pend_stage = 0;
  int c_mt = g0 / nk, c_kt = g0 - c_mt * nk;  // tile and k-tile of iteration g
  int stored = 0;                              // stores issued at the end of the last iteration
  auto tail = [&]() {
    stored = 0;
    if (c_kt == nk - 1 || g == last) {
      const int slot = j - c_mt * nk / Lshare;  // this segment's C block
      gm_store(L, acc, C + slot * slot_stride, ldc, c * GM_BN, c_mt * GM_BM, false);
      stored = 16;
      gm_zero(acc);
    }
    if (++c_kt == nk) {
      c_kt = 0;
      ++c_mt;
    }
  };
  gm_iteration<true>(L, gm_smem, acc, f0, f1, stage, pend_stage, stored, src, next);
  tail();
  first = false;
  for (g = g0 + 1; g < g1; g++) {
    gm_iteration<false>(L, gm_smem, acc, f0, f1, stage, pend_stage, stored, src, next);
    tail();
  }
  // direct loads and stores in flight must finish before the block ends
  __builtin_amdgcn_s_waitcnt(gm_vmcnt(0));
}

// ---------------------------------------------------------------- host side
struct GemmPlan {
  bool stream = false;
  int ks = 1;      // split grid: K slices
  int grid = 0;    // stream grid: blocks
  int share = 0;   // stream grid: k-tiles per block
  int slices = 1;  // C blocks the consumer sums
};

// Calls f(std::integral_constant<int, NS>) for the slice counts a plan can
// produce (ns in {1, 2, 4, 8}), so the consumer kernels sum a compile-time
// number of slices; false for any other count.
template <typename F>
inline bool gm_with_slices(int ns, F &&f) {
  switch (ns) {
    case 1: f(std::integral_constant<int, 1>{}); return true;
    case 2: f(std::integral_constant<int, 2>{}); return true;
    case 4: f(std::integral_constant<int, 4>{}); return true;
    case 8: f(std::integral_constant<int, 8>{}); return true;
    default: return false;
  }
}

// Consumer slice count of a balanced grid with per_col shares of L k-tiles
// per column: the most segments any tile is cut into, rounded up to 1, 2, 4
// or 8 (0: more than 8)
inline int gemm_stream_slices(int m_tiles, int nk, int L) {
  int most = 1;
  for (int mt = 0; mt < m_tiles; mt++) {
    const int segs = (mt * nk + nk - 1) / L - mt * nk / L + 1;
    if (segs > most) most = segs;
  }
  return most == 1 ? 1 : most == 2 ? 2 : most <= 4 ? 4 : most <= 8 ? 8 : 0;
}

// cus: the device's compute units (8 XCDs).  Shapes must satisfy
// M % 256 == 0, nt % 64 == 0, K % 64 == 0.
inline GemmPlan gemm_plan(int M, int K, int nt, int cus) {
  GemmPlan p;
  const int m_tiles = M / GM_BM, n_tiles = nt / GM_BN, tiles = m_tiles * n_tiles, nk = K / GM_BK;
  if (tiles > cus) {
    const int per_col = 8 * ((cus / 8) / n_tiles);  // balanced grid: shares per column tile
    if (per_col >= 8 && m_tiles >= per_col) {
      p.stream = true;
      p.grid = per_col * n_tiles;
      p.share = (m_tiles * nk + per_col - 1) / per_col;
      p.slices = gemm_stream_slices(m_tiles, nk, p.share);
      return p;
    }
    return p;  // split grid, K whole, several rounds
  }
  // At most one block per CU: K split in KS slices.  (The balanced grid on
  // all CUs, with a tile cut into up to 8 segments, measured slower for these
  // shapes: QKV, O and down of the 256-token prompt took 2-5 us more each.)
  while (p.ks < 8 && tiles * p.ks * 2 <= cus && (nk % (p.ks * 2)) == 0 && nk / (p.ks * 2) >= 2) p.ks *= 2;
  p.slices = p.ks;
  return p;
}

// both kernels use 144 KB of dynamic LDS
inline hipError_t gemm_setup() {
  hipError_t e = hipFuncSetAttribute((const void *)gemm_split_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                     GM_LDS);
  if (e != hipSuccess) return e;
  return hipFuncSetAttribute((const void *)gemm_stream_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, GM_LDS);
}

inline void gemm_launch(const GemmPlan &p, hipStream_t st, const uint16_t *W, int M, int K, const uint16_t *B,
                        int nt, float *C) {
  if (p.stream)
    hipLaunchKernelGGL(gemm_stream_kernel, dim3(p.grid), dim3(256), GM_LDS, st, W, M, K, B, nt, C, M, p.share,
                       p.slices);
  else
    hipLaunchKernelGGL(gemm_split_kernel, dim3((M / GM_BM) * (nt / GM_BN), p.ks), dim3(256), GM_LDS, st, W, M, K,
                       B, nt, C, M);
}

}  // namespace vx
