// vx_engine.hip -- host side of libvoxtral_amd.so: the C ABI declared in
// include/voxtral_engine.h.  Replaces the WebGPU dispatch layer and
// orchestration of src/engine.ts (backboneStep :814-1042, fmForward
// :1240-1380, generate :2416-2616) with HIP launches on one stream, the
// per-step kernel sequence captured once into hipGraphs.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <numeric>
#include <string>
#include <vector>

#include "../../include/voxtral_engine.h"
#include "vx_kernels.h"
#include "vx_prefill.h"
#include "vx_codec.h"
#include "vx_gemm.h"
#include "vx_loader.h"
#include "vx_tokenizer.h"

#include <fcntl.h>
#include <unistd.h>

using namespace vx;

namespace {

char g_create_error[512] = "";

struct LayerW {
  uint16_t *wqkv = nullptr, *wo = nullptr, *w1 = nullptr, *w3 = nullptr, *w2 = nullptr,
           *attn_norm = nullptr, *ffn_norm = nullptr;
};

struct Slot {
  uint16_t *ptr;
  std::vector<int64_t> shape;
  size_t numel;
  bool is_norm;  // gains and scales: synthetic weights centred on 1
  bool loaded;
};

// codec decoder weights (src/engine.ts:700-770).  wq, wk, wv are adjacent
// (wqkv), and so are w1, w3 (w13), so each pair is one stacked GEMM.
struct CodecLayerW {
  uint16_t *attn_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr, *wqkv = nullptr,
           *wo = nullptr, *attn_scale = nullptr, *ffn_norm = nullptr, *w13 = nullptr,
           *w2 = nullptr, *ffn_scale = nullptr;
};
struct CodecW {
  uint16_t *in_w = nullptr, *in_g = nullptr, *out_w = nullptr, *out_g = nullptr,
           *cb_sum = nullptr, *cb_usage = nullptr;
  uint16_t *up_w[CX_STAGES - 1] = {}, *up_g[CX_STAGES - 1] = {};
  CodecLayerW L[CX_STAGES][CX_LPS];
};

// FNV-1a 64 of "fm.noise": generator stream of the per-frame FM noise
constexpr uint64_t kNoiseStream = 0x45237962ac6f43f0ull;

constexpr size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

}  // namespace

struct vx_tokenizer {
  vx::BpeVocab vocab;
};

struct vx_engine {
  vx_config cfg;
  int max_seq = 0;
  hipStream_t st = nullptr;
  std::string err;

  // weights
  void *warena = nullptr;
  std::vector<LayerW> L, FL;
  uint16_t *tok_emb = nullptr, *audio_emb = nullptr, *final_norm = nullptr;
  uint16_t *fm_in = nullptr, *fm_llm = nullptr, *fm_time = nullptr, *fm_norm = nullptr,
           *fm_sem = nullptr, *fm_ac = nullptr;
  std::map<std::string, Slot> slots;

  // KV cache [layer][K|V][NKV][max_seq][HD], f32 (default) or f16 elements
  void *kv = nullptr;
  int kv_f32 = 1;
  size_t kv_elem = 4;

  // activations
  void *aarena = nullptr;
  float *x = nullptr, *q = nullptr, *attn = nullptr, *act = nullptr, *normed = nullptr,
        *logits = nullptr, *part = nullptr, *layer_stage = nullptr;
  // the state the previous frame left (multi_codebook_kernel saves it)
  float *x_prev = nullptr, *normed_prev = nullptr, *logits_prev = nullptr;
  // launch timeline of one step: [6 * n_layers + 1][TS_BLOCKS][start, end] wall-clock stamps
  unsigned long long *timeline = nullptr;
  int *pos = nullptr, *frame = nullptr;
  uint32_t *sem_code = nullptr, *codes = nullptr, *argmax_res = nullptr;
  uint64_t *noise_seed = nullptr;
  float *inv_freq = nullptr;  // rope inverse frequencies [HD/2]
  float *fm_seq = nullptr, *fm_q = nullptr, *fm_k = nullptr, *fm_v = nullptr, *fm_attn = nullptr,
        *fm_act = nullptr, *fm_llm_out = nullptr, *sem_logits = nullptr, *tproj = nullptr,
        *xh = nullptr, *vel = nullptr, *noise = nullptr, *time_embed = nullptr;
  // the last FM layer's acoustic-projection partials per 12-row tile
  float *ac_part = nullptr, *ac_ssq = nullptr;
  bool tproj_ready = false;
  // FM layer matrices in the MFMA A-operand order (pack_mfma_a_kernel), and
  // the packed inputs / sums of squares the FM GEMMs hand to each other
  void *fm_parena = nullptr;
  std::vector<LayerW> FP;
  bool fm_packed_ready = false;
  h8 *fm_b_attn = nullptr, *fm_b_o = nullptr, *fm_b_ffn = nullptr, *fm_b_act = nullptr;
  float *fm_ssq_attn = nullptr, *fm_ssq_ffn = nullptr;
  // batched prefill (vx_prefill.h): chunk activations, packed GEMM input,
  // GEMM output, the chunk's token ids and voice rows
  void *pf_arena = nullptr;
  float *pf_x = nullptr, *pf_q = nullptr, *pf_c = nullptr,
        *pf_voice = nullptr;
  h8 *pf_b = nullptr;
  int32_t *pf_tok = nullptr;
  int pf_chunk = PF_MAXT;  // tokens per prefill chunk (multiple of 128)

  int host_pos = 0;
  hipGraphExec_t step_exec = nullptr, hold_exec = nullptr, feedback_exec = nullptr,
                 frame_exec = nullptr, timeline_exec = nullptr,
                 fm_greedy_exec = nullptr, fm_plain_exec = nullptr;
  bool use_graphs = true;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  // device top-p: its uniform stream and (top_p, temperature); a logits
  // buffer for vx_sample_top_p; pinned per-frame readback slots
  uint64_t *rng_state = nullptr;
  double *tp_params = nullptr;
  float *tp_logits = nullptr;
  uint32_t *h_frame = nullptr;  // [2][1 + NAC], pinned, written by the frame's last kernels
  uint32_t *d_frame = nullptr;  // h_frame's device address
  hipEvent_t ev_frame[2] = {nullptr, nullptr};
  hipGraphExec_t fm_topp_exec = nullptr, frame_topp_exec = nullptr;

  // codec decoder: weights; derived operands (normalised codebook, conv
  // weights in GEMM order, weight-norm scales), rebuilt after weight loads;
  // per-decode buffers sized for cx_cap frames
  bool codec_on = false, codec_ready = false;
  CodecW cw;
  void *cx_parena = nullptr;
  uint16_t *cx_cb = nullptr, *cx_ain = nullptr, *cx_aout = nullptr, *cx_aup[CX_STAGES - 1] = {};
  float *cx_rs_in = nullptr, *cx_rs_out = nullptr, *cx_s_up[CX_STAGES - 1] = {};
  void *cx_arena = nullptr;
  int cx_cap = 0;
  float *cx_x = nullptr, *cx_x2 = nullptr, *cx_q = nullptr, *cx_k = nullptr, *cx_v = nullptr,
        *cx_attn = nullptr, *cx_c = nullptr, *cx_audio = nullptr;
  h8 *cx_b = nullptr;
  uint32_t *cx_sem = nullptr, *cx_ac = nullptr;
  int cx_chunk = CX_MAXT;  // tokens per codec GEMM chunk (multiple of 128)

  bool gemm_ready = false;
  int cus = 0;  // compute units (prefill GEMM grids)

  void weights_changed() {
    tproj_ready = false;
    fm_packed_ready = false;
    codec_ready = false;
  }

  void *kc(int l) const { return (char *)kv + (size_t)(2 * l) * NKV * max_seq * HD * kv_elem; }
  void *vc(int l) const { return (char *)kv + (size_t)(2 * l + 1) * NKV * max_seq * HD * kv_elem; }
  int nsteps() const { return cfg.nfe - 1; }
};

// ----------------------------------------------------------------- errors
static int fail(vx_engine *e, int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (e)
    e->err = buf;
  else
    snprintf(g_create_error, sizeof g_create_error, "%s", buf);
  return code;
}

#define HIPCHK(e, call)                                                            \
  do {                                                                             \
    hipError_t _s = (call);                                                        \
    if (_s != hipSuccess)                                                          \
      return fail((e), VX_E_DEVICE, "%s failed: %s", #call, hipGetErrorString(_s)); \
  } while (0)

#define LAUNCHCHK(e)                                                                  \
  do {                                                                                \
    hipError_t _s = hipGetLastError();                                                \
    if (_s != hipSuccess)                                                             \
      return fail((e), VX_E_DEVICE, "kernel launch failed: %s", hipGetErrorString(_s)); \
  } while (0)

static uint64_t fnv1a(const char *s) {
  uint64_t h = 0xcbf29ce484222325ull;
  for (; *s; s++) {
    h ^= (unsigned char)*s;
    h *= 0x100000001b3ull;
  }
  return h;
}

// ------------------------------------------------------- kernel launchers
namespace {

// Launch shapes.  Rows per block = WAVES * RPW (SwiGLU: pairs = WAVES*RPW/2).
constexpr int W4 = 4;

template <int NB, int WAVES, int RPW, int EPI, bool NORM, int K, int KT>
void launch_gemv(hipStream_t st, const GemvArgs &a) {
  constexpr int units = WAVES * (EPI == EPI_SWIGLU ? RPW / 2 : RPW);
  const int grid = (a.M + units - 1) / units;
  hipLaunchKernelGGL((gemv_kernel<NB, WAVES, RPW, EPI, NORM, K, KT>), dim3(grid),
                     dim3(WAVES * 64), 0, st, a.W, a.W2, a.x, a.norm_w, a.out, a);
}

GemvArgs gargs(const uint16_t *W, const float *x, int xs, float *out, int os, int M) {
  GemvArgs a;
  memset(&a, 0, sizeof a);
  a.W = W;
  a.x = x;
  a.xs = xs;
  a.out = out;
  a.os = os;
  a.M = M;
  return a;
}

}  // namespace


// FM GEMM launch: `rows` output rows in tiles of FTR, RG tiles per block.
template <int EPI, int K, int RG, int KS, int P, bool KEEP = false>
void launch_gemm6(hipStream_t st, const Gemm6Args &a, int rows) {
  hipLaunchKernelGGL((gemm6_kernel<EPI, K, RG, KS, P, KEEP>), dim3(rows / (FTR * RG)), dim3(RG * KS * 64),
                     0, st, a.W, a.W2, a.B, a.ssq, a.out, a);
}
// Launch shapes of the four FM GEMMs <RG, KS, P>, picked on the whole frame
// loop.
#define FM_GEMM_QKV (launch_gemm6<EPI_QKV, DIM, 1, 4, 8>)
#define FM_GEMM_O (launch_gemm6<EPI_RESID, QD, 1, 8, 16>)
#define FM_GEMM_O_KEEP (launch_gemm6<EPI_RESID, QD, 1, 8, 16, true>)
#define FM_GEMM_GATEUP (launch_gemm6<EPI_SWIGLU, DIM, 1, 1, 16>)
#define FM_GEMM_DOWN (launch_gemm6<EPI_RESID, HID, 1, 12, 12>)
// 12-row tiles divide every FM matrix into a multiple of 256 tiles
static_assert(QKV_ROWS % (256 * FTR) == 0 && DIM % (256 * FTR) == 0 && HID % (256 * FTR) == 0 &&
                  DIM / FTR <= SSQ_MAX && DIM % 256 == 0,
              "FM GEMM tiles");

// decode attention partials: one block per (split, KV head)
static dim3 attn_grid() { return dim3(ATTN_SPLITS * NKV); }

// Streaming GEMV launch: M units split exactly into blocks of WAVES*UPW.
template <int WAVES, int UPW, int UPG, int EPI, bool NORM, int K, int D = 2>
void launch_gemv1(hipStream_t st, const GemvArgs &a) {
  constexpr int per_block = WAVES * UPW;
  hipLaunchKernelGGL((gemv1_kernel<WAVES, UPW, UPG, EPI, NORM, K, D>), dim3(a.M / per_block),
                     dim3(WAVES * 64), 0, st, a.W, a.W2, a.x, a.norm_w, a.out, a.ts, a);
}
// Backbone GEMV launch shapes (waves per block, one unit per wave), picked
// by a sweep over 4-16 waves per block on the decode step.
#define BB_GEMV_QKV (launch_gemv1<6, 1, 1, EPI_QKV_ROPE, true, DIM, 1>)
#define BB_GEMV_O (launch_gemv1<12, 1, 1, EPI_RESID, false, QD, 1>)
#define BB_GEMV_GATEUP (launch_gemv1<12, 1, 1, EPI_SWIGLU, true, DIM, 1>)
#define BB_GEMV_DOWN (launch_gemv1<6, 1, 1, EPI_RESID, false, HID, 1>)
// unit counts of the backbone GEMVs must split into whole blocks
static_assert((QKV_ROWS / 2) % 6 == 0 && DIM % 12 == 0 && HID % 12 == 0 && DIM % 6 == 0,
              "launch shapes");

// One backbone layer: 6 launches (norm + QKV + rope + KV write | attention
// partials | attention combine | O + residual | norm + gate/up + SwiGLU |
// down + residual).
// ts: the step's launch timeline (vx_debug_timeline), or null; launch k of
// layer l (0 QKV, 1 attention partials, 2 combine, 3 O, 4 gate/up, 5 down)
// writes its blocks' stamps to slot 6 l + k (2 * TS_BLOCKS values).
static void enqueue_layer(vx_engine *e, int l, int only = -1, unsigned long long *ts = nullptr) {
  const LayerW &W = e->L[l];
  hipStream_t st = e->st;
  auto slot = [&](int k) { return ts ? ts + (size_t)2 * TS_BLOCKS * (6 * l + k) : nullptr; };
  if (only < 0 || only == VX_KERNEL_QKV) {
    GemvArgs a = gargs(W.wqkv, e->x, DIM, e->q, 0, QKV_ROWS / 2);
    a.norm_w = W.attn_norm;
    a.eps = e->cfg.norm_eps;
    a.pos = e->pos;
    a.kc = e->kc(l);
    a.vc = e->vc(l);
    a.kv_f32 = e->kv_f32;
    a.max_seq = e->max_seq;
    a.inv_freq = e->inv_freq;
    a.ts = slot(0);
    BB_GEMV_QKV(st, a);
  }
  if (only < 0 || only == VX_KERNEL_ATTN) {
    AttnArgs a{e->q, e->kc(l), e->vc(l), e->pos, e->max_seq, e->part, e->attn, slot(1)};
    if (e->kv_f32)
      hipLaunchKernelGGL(attn_partial_kernel<float>, attn_grid(), dim3(256), KvRing<float>::LDS, st, a.pos,
                         a.kc, a.vc, a.q, a.ts, a);
    else
      hipLaunchKernelGGL(attn_partial_kernel<uint16_t>, attn_grid(), dim3(256), KvRing<uint16_t>::LDS, st,
                         a.pos, a.kc, a.vc, a.q, a.ts, a);
    hipLaunchKernelGGL(attn_combine_kernel, dim3(NH), dim3(64), 0, st, e->part, e->attn, slot(2));
  }
  if (only < 0 || only == VX_KERNEL_OPROJ) {
    GemvArgs a = gargs(W.wo, e->attn, QD, e->x, 0, DIM);
    a.ts = slot(3);
    BB_GEMV_O(st, a);
  }
  if (only < 0 || only == VX_KERNEL_GATEUP) {
    GemvArgs a = gargs(W.w1, e->x, DIM, e->act, 0, HID);
    a.W2 = W.w3;
    a.norm_w = W.ffn_norm;
    a.eps = e->cfg.norm_eps;
    a.ts = slot(4);
    BB_GEMV_GATEUP(st, a);
  }
  if (only < 0 || only == VX_KERNEL_DOWN) {
    GemvArgs a = gargs(W.w2, e->act, HID, e->x, 0, DIM);
    a.ts = slot(5);
    BB_GEMV_DOWN(st, a);
  }
}

static void enqueue_backbone_at(vx_engine *e, bool advance, unsigned long long *ts = nullptr) {
  for (int l = 0; l < e->cfg.n_layers; l++) enqueue_layer(e, l, -1, ts);
  hipLaunchKernelGGL(final_norm_kernel, dim3(1), dim3(1024), 0, e->st, e->x, e->final_norm,
                     e->cfg.norm_eps, e->normed, advance ? e->pos : nullptr,
                     ts ? ts + (size_t)2 * TS_BLOCKS * 6 * e->cfg.n_layers : nullptr);
}
static void enqueue_backbone(vx_engine *e) { enqueue_backbone_at(e, true); }
static void enqueue_backbone_hold(vx_engine *e) { enqueue_backbone_at(e, false); }
// the held step with its launch timeline recorded (vx_debug_timeline)
static void enqueue_backbone_timeline(vx_engine *e) { enqueue_backbone_at(e, false, e->timeline); }

__global__ void copy_dim_kernel(const float *src, float *dst) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < DIM) dst[i] = src[i];
}
// A step whose input embedding is the previous step's W.normed, through the
// precomputed-embedding path (src/engine.ts:847-854): a prompt's decode tail
// fed with each frame's output hidden state.
static void enqueue_backbone_feedback(vx_engine *e) {
  hipLaunchKernelGGL(copy_dim_kernel, dim3(DIM / 256), dim3(256), 0, e->st, e->normed, e->x);
  enqueue_backbone_at(e, true);
}

static void enqueue_lm_head(vx_engine *e) {
  GemvArgs a = gargs(e->tok_emb, e->normed, DIM, e->logits, 0, e->cfg.vocab_size);
  launch_gemv<1, W4, 2, EPI_PLAIN, false, DIM, DIM>(e->st, a);
  hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(256), 0, e->st, e->logits, e->cfg.vocab_size, 0,
                     e->argmax_res);
}

// Before an FM pass: the time-projection table of the nfe-1 timesteps and
// the MFMA-order copies of the FM layer matrices (redone after any load).
static int ensure_tproj(vx_engine *e) {
  if (!e->fm_packed_ready) {
    auto pack = [&](const uint16_t *src, uint16_t *dst, int M, int K) {
      hipLaunchKernelGGL(pack_mfma_a_kernel, dim3(2048), dim3(256), 0, e->st, src, dst, M, K);
    };
    for (size_t l = 0; l < e->FL.size(); l++) {
      const LayerW &W = e->FL[l], &P = e->FP[l];
      pack(W.wqkv, P.wqkv, QKV_ROWS, DIM);
      pack(W.wo, P.wo, DIM, QD);
      pack(W.w1, P.w1, HID, DIM);
      pack(W.w3, P.w3, HID, DIM);
      pack(W.w2, P.w2, DIM, HID);
    }
    LAUNCHCHK(e);
    e->fm_packed_ready = true;
  }
  if (e->tproj_ready) return VX_OK;
  for (int s = 0; s < e->nsteps(); s++) {
    float t = (float)((double)s / (double)(e->cfg.nfe - 1));
    hipLaunchKernelGGL(time_embed_kernel, dim3((DIM / 2 + 255) / 256), dim3(256), 0, e->st,
                       e->time_embed, t);
    GemvArgs a = gargs(e->fm_time, e->time_embed, DIM, e->tproj + (size_t)s * DIM, 0, DIM);
    launch_gemv<1, W4, 2, EPI_PLAIN, false, DIM, DIM>(e->st, a);
  }
  LAUNCHCHK(e);
  e->tproj_ready = true;
  return VX_OK;
}

// The FM kernels of one Euler step, by kind (also timed one by one).
enum FmKernel { FMK_QKV, FMK_ATTN, FMK_O, FMK_GATEUP, FMK_DOWN };

// Kernel k of FM layer l.  nssq_attn: partial sums of squares of the QKV
// input (DIM / 256 from the step's input kernel for layer 0, DIM / FTR from
// the previous layer's down GEMM).
static void enqueue_fm_kernel(vx_engine *e, int l, int k, int nssq_attn) {
  hipStream_t st = e->st;
  const LayerW &W = e->FL[l], &P = e->FP[l];
  const bool last = l + 1 == e->cfg.fm_layers;
  switch (k) {
    case FMK_QKV: {  // RMSNorm + QKV (no rope: src/engine.ts:1108)
      Gemm6Args a{};
      a.W = P.wqkv;
      a.B = e->fm_b_attn;
      a.ssq = e->fm_ssq_attn;
      a.nssq = nssq_attn;
      a.eps = 1e-5f;
      a.out = e->fm_q;
      a.out_k = e->fm_k;
      a.out_v = e->fm_v;
      FM_GEMM_QKV(st, a, QKV_ROWS);
      break;
    }
    case FMK_ATTN:
      hipLaunchKernelGGL(fm_attn_kernel, dim3(NH, 2), dim3(64), 0, st, e->fm_q, e->fm_k, e->fm_v,
                         e->fm_attn, e->fm_b_o);
      break;
    case FMK_O: {  // O + residual; hands norm(x) * ffn gains to gate/up
      Gemm6Args a{};
      a.W = P.wo;
      a.B = e->fm_b_o;
      a.out = e->fm_seq;
      a.os = DIM;
      a.Bn = e->fm_b_ffn;
      a.gn = W.ffn_norm;
      a.ssq_out = e->fm_ssq_ffn;
      // Layer 0's O matrix (25 MB, about 3.1 MB per XCD's 4 MB L2) is read
      // with plain loads, so much of it is still in L2 at the next Euler
      // step (6.3 against 7.5 us per launch); every other weight stream is
      // non-temporal.  Only one FM matrix fits.
      if (l == 0)
        FM_GEMM_O_KEEP(st, a, DIM);
      else
        FM_GEMM_O(st, a, DIM);
      break;
    }
    case FMK_GATEUP: {  // RMSNorm + gate/up + SwiGLU; hands the activation to down
      Gemm6Args a{};
      a.W = P.w1;
      a.W2 = P.w3;
      a.B = e->fm_b_ffn;
      a.ssq = e->fm_ssq_ffn;
      a.nssq = DIM / FTR;
      a.eps = 1e-5f;
      a.out = e->fm_act;
      a.os = HID;
      a.Bn = e->fm_b_act;
      FM_GEMM_GATEUP(st, a, HID);
      break;
    }
    default: {  // down + residual; hands norm(x) * next attention gains to the next layer
      Gemm6Args a{};
      a.W = P.w2;
      a.B = e->fm_b_act;
      a.out = e->fm_seq;
      a.os = DIM;
      if (!last) {
        a.Bn = e->fm_b_attn;
        a.gn = e->FL[l + 1].attn_norm;
        a.ssq_out = e->fm_ssq_attn;
      } else {  // the velocity's final norm + acoustic projection, split per tile
        a.acw = e->fm_ac;
        a.acg = e->fm_norm;
        a.ac_part = e->ac_part;
        a.ac_ssq = e->ac_ssq;
      }
      FM_GEMM_DOWN(st, a, DIM);
      break;
    }
  }
}

// Start of Euler step s (x_s, the input projection, both CFG sequences).
// The input kernel of Euler step s.  noise_src: x_0 (step 0), or null for
// the device generator (seed, kNoiseStream, frame counter).  sem_mask >= 0:
// step 0 also takes the argmax of the semantic logits into sem_code, with
// argmax_kernel's mask (8194: the greedy code's valid range; 0: unmasked).
static void enqueue_fm_step_in(vx_engine *e, int s, const float *noise_src, int sem_mask = -1) {
  const float alpha = e->cfg.cfg_alpha;
  const float dt = (float)(1.0 / (double)(e->cfg.nfe - 1));
  FmStepArgs fa{e->xh,      e->vel,    e->ac_part, e->ac_ssq, e->fm_in,
                e->tproj + (size_t)s * DIM, e->fm_llm_out, e->fm_seq, s, alpha, dt, noise_src,
                e->noise_seed, kNoiseStream, e->frame,
                e->fm_b_attn, e->FL[0].attn_norm, e->fm_ssq_attn,
                e->sem_logits, sem_mask, e->sem_code};
  const bool argmax = s == 0 && sem_mask >= 0;
  hipLaunchKernelGGL(fm_step_in_kernel, dim3(DIM / 256 + (argmax ? 1 : 0)), dim3(256), 0, e->st, fa.w_in,
                     fa.ac_part, fa.ac_ssq, fa.xh, fa);
}

// fmForward with CFG batched: 6 vectors (2 branches x 3 positions) share
// every weight read; time projections come from the precomputed table.
// noise_src: device f32[36] holding x_0, or null for the device generator.
static void enqueue_fm(vx_engine *e, const float *noise_src, bool greedy_code) {
  hipStream_t st = e->st;
  const float alpha = e->cfg.cfg_alpha;
  const float dt = (float)(1.0 / (double)(e->cfg.nfe - 1));
  {  // llm_projection + semantic head: the stacked [3072 + 8320][3072] rows
     // (fm_llm, fm_sem) into the adjacent fm_llm_out, sem_logits
    GemvArgs a = gargs(e->fm_llm, e->normed, DIM, e->fm_llm_out, 0, DIM + SEMV);
    launch_gemv1<8, 1, 1, EPI_PLAIN, false, DIM, 1>(st, a);
  }
  for (int s = 0; s < e->nsteps(); s++) {
    // step 0 also takes the unmasked tree argmax (W.semantic_argmax), or the
    // masked one for greedy codes
    enqueue_fm_step_in(e, s, noise_src, s == 0 ? (greedy_code ? 8194 : 0) : -1);
    for (int l = 0; l < e->cfg.fm_layers; l++)
      for (int k = FMK_QKV; k <= FMK_DOWN; k++) enqueue_fm_kernel(e, l, k, l == 0 ? DIM / 256 : DIM / FTR);
    // the step's velocities (final norm of position 0 of each branch ->
    // acoustic_out) are finished from the partials by the next step's input
    // kernel, and for the last step by fm_finish
  }
  hipLaunchKernelGGL(fm_finish_kernel, dim3(1), dim3(256), 0, st, e->xh, e->vel, e->ac_part, e->ac_ssq,
                     e->nsteps() - 1, alpha, dt, e->codes, e->cfg.acoustic_levels, e->frame, e->sem_code,
                     e->d_frame);
}

// ------------------------------------------------------------------ graphs
static int capture(vx_engine *e, hipGraphExec_t *out, void (*body)(vx_engine *)) {
  hipGraph_t g;
  HIPCHK(e, hipStreamBeginCapture(e->st, hipStreamCaptureModeThreadLocal));
  body(e);
  hipError_t cap = hipStreamEndCapture(e->st, &g);
  if (cap != hipSuccess) return fail(e, VX_E_DEVICE, "graph capture: %s", hipGetErrorString(cap));
  hipError_t s = hipGraphInstantiate(out, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (s != hipSuccess) return fail(e, VX_E_DEVICE, "graph instantiate: %s", hipGetErrorString(s));
  return VX_OK;
}

// FM part of a frame: seeded device noise, then fmForward; greedy stores
// the masked argmax as the device semantic code (no host round trip).
// x_0 from the device generator, drawn by the first Euler step's kernel
static void fm_greedy_body(vx_engine *e) { enqueue_fm(e, nullptr, true); }
static void fm_plain_body(vx_engine *e) { enqueue_fm(e, nullptr, false); }
// FM, then the semantic code by device top-p (masked, src/engine.ts:2556-2567)
static void fm_topp_body(vx_engine *e) {
  fm_plain_body(e);
  hipLaunchKernelGGL(topp_sample_kernel, dim3(1), dim3(TP_NT), 0, e->st, e->sem_logits, SEMV, 8194,
                     e->tp_params, e->rng_state, e->sem_code, e->frame, e->d_frame);
}
// A frame's first kernel embeds the previous frame's codes and saves the
// state that frame left (FrameSave), for generate()'s EOS rollback.
static void enqueue_frame_embed(vx_engine *e) {
  const FrameSave sv{e->x_prev, e->normed_prev, e->logits_prev, e->normed, e->sem_logits};
  hipLaunchKernelGGL(multi_codebook_kernel, dim3(DIM / 256), dim3(256), 0, e->st, e->audio_emb,
                     e->sem_code, e->codes, e->x, sv);
}
static void frame_body(vx_engine *e) {
  enqueue_frame_embed(e);
  enqueue_backbone(e);
  fm_greedy_body(e);
}
static void frame_topp_body(vx_engine *e) {
  enqueue_frame_embed(e);
  enqueue_backbone(e);
  fm_topp_body(e);
}

// Runs one captured sequence: replays its hipGraph (captured on first use),
// or, when graphs are off (VX_NO_GRAPH=1, e.g. under a kernel tracer),
// enqueues the same kernels directly.
static int run_seq(vx_engine *e, hipGraphExec_t *slot, void (*body)(vx_engine *)) {
  if (!e->use_graphs) {
    body(e);
    LAUNCHCHK(e);
    return VX_OK;
  }
  if (!*slot) {
    int rc = capture(e, slot, body);
    if (rc) return rc;
  }
  HIPCHK(e, hipGraphLaunch(*slot, e->st));
  return VX_OK;
}
static int run_step(vx_engine *e) {
  return run_seq(e, &e->step_exec, enqueue_backbone);
}
static int run_step_hold(vx_engine *e) {
  return run_seq(e, &e->hold_exec, enqueue_backbone_hold);
}

// ---------------------------------------------------------------- helpers
__global__ void set_int_kernel(int *p, int v) { *p = v; }
__global__ void set_u32_kernel(uint32_t *p, const uint32_t v0) { *p = v0; }

static int check_ready(vx_engine *e) {
  for (auto &kv : e->slots)
    if (!kv.second.loaded) return fail(e, VX_E_STATE, "Missing weight: %s", kv.first.c_str());
  return VX_OK;
}

static int prepare_input(vx_engine *e, int32_t token, int32_t mode, const float *pre) {
  if (e->host_pos >= e->max_seq)
    return fail(e, VX_E_RANGE, "position %d reaches max_seq_len %d", e->host_pos, e->max_seq);
  switch (mode) {
    case VX_EMBED_TOKEN:
      if (token < 0 || token >= e->cfg.vocab_size)
        return fail(e, VX_E_INVALID, "token %d outside vocab", token);
      hipLaunchKernelGGL(embed_row_kernel, dim3(DIM / 256), dim3(256), 0, e->st, e->tok_emb, token,
                         e->x);
      break;
    case VX_EMBED_AUDIO:
      if (token < 0 || token >= e->cfg.audio_vocab)
        return fail(e, VX_E_INVALID, "audio token %d outside table", token);
      hipLaunchKernelGGL(embed_row_kernel, dim3(DIM / 256), dim3(256), 0, e->st, e->audio_emb,
                         token, e->x);
      break;
    case VX_EMBED_PRECOMPUTED:
      if (!pre) return fail(e, VX_E_INVALID, "precomputed embedding is NULL");
      HIPCHK(e, hipMemcpyAsync(e->x, pre, DIM * sizeof(float), hipMemcpyHostToDevice, e->st));
      break;
    case VX_EMBED_CODES:
      hipLaunchKernelGGL(multi_codebook_kernel, dim3(DIM / 256), dim3(256), 0, e->st, e->audio_emb,
                         e->sem_code, e->codes, e->x, FrameSave{});
      break;
    default:
      return fail(e, VX_E_INVALID, "bad embed mode %d", mode);
  }
  LAUNCHCHK(e);
  return VX_OK;
}

// ------------------------------------------ allocation-free top-p staging
// vx_sample_top_p_noalloc stages its operands in this file-scope device
// array instead of an engine's allocation: the caller's logits (at most
// TP_MAXN), the (top_p, temperature) pair, the splitmix64 state and the
// picked code.  Every GPU holds its own copy until the process ends.  Host
// code never passes `scratch` itself to a kernel or a copy (in host code the
// name is only a stand-in): the device address comes from
// hipGetSymbolAddress, looked up once per device with that device current.
namespace {
constexpr size_t NA_LOGITS = 0;
constexpr size_t NA_PARAMS = NA_LOGITS + (size_t)TP_MAXN * 4;  // 2 doubles
constexpr size_t NA_STATE = NA_PARAMS + 16;                    // u64
constexpr size_t NA_CODE = NA_STATE + 8;                       // u32
constexpr size_t NA_BYTES = (NA_CODE + 4 + 255) & ~size_t(255);
static_assert(NA_PARAMS % 8 == 0 && NA_STATE % 8 == 0, "staging alignment");
constexpr int NA_MAX_DEVICES = 64;
std::mutex g_na_mu;
char *g_na_ptr[NA_MAX_DEVICES] = {};
// held by a call for its whole use of the device's array (copies in, kernel,
// copies out, sync): calls from threads of one process take turns
std::mutex g_na_call_mu[NA_MAX_DEVICES];
}  // namespace
static __device__ __align__(256) unsigned char scratch[NA_BYTES];

// the array's address on the current device (looked up on the first call
// there) and that device's index; nullptr and g_create_error set on failure
static char *noalloc_scratch(int *dev_out) {
  int dev = -1;
  hipError_t s = hipGetDevice(&dev);
  if (s != hipSuccess || dev < 0 || dev >= NA_MAX_DEVICES) {
    fail(nullptr, VX_E_DEVICE, "no current HIP device (%s)", hipGetErrorString(s));
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_na_mu);
  if (!g_na_ptr[dev]) {
    void *p = nullptr;
    s = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (s != hipSuccess || !p) {
      fail(nullptr, VX_E_DEVICE, "hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(s));
      return nullptr;
    }
    g_na_ptr[dev] = (char *)p;
  }
  *dev_out = dev;
  return g_na_ptr[dev];
}

// ================================================================ C ABI
extern "C" {

int vx_config_default(vx_config *c) {
  if (!c) return VX_E_INVALID;
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
  c->kv_f16 = 0;
  c->codec = 1;
  return VX_OK;
}

const char *vx_last_error(const vx_engine *e) { return e ? e->err.c_str() : g_create_error; }

static void add_slot(vx_engine *e, const std::string &name, uint16_t *ptr,
                     std::vector<int64_t> shape, bool is_norm) {
  size_t n = 1;
  for (auto s : shape) n *= (size_t)s;
  e->slots[name] = Slot{ptr, shape, n, is_norm, false};
}

int vx_create(const vx_config *cfg_in, int32_t max_seq, vx_engine **out) {
  if (!out) return fail(nullptr, VX_E_INVALID, "out is NULL");
  *out = nullptr;
  vx_config cfg;
  vx_config_default(&cfg);
  if (cfg_in) cfg = *cfg_in;
  if (cfg.dim != DIM || cfg.head_dim != HD || cfg.n_heads != NH || cfg.n_kv_heads != NKV ||
      cfg.hidden_dim != HID || cfg.n_acoustic_out != NAC || cfg.semantic_vocab != SEMV)
    return fail(nullptr, VX_E_INVALID,
                "unsupported shape: the kernels are built for dim 3072, 32/8 heads of 128, "
                "FFN 9216, 36 acoustic dims, semantic vocab 8320");
  if (cfg.n_layers < 1 || cfg.n_layers > 64 || cfg.fm_layers < 1 || cfg.fm_layers > 16 ||
      cfg.nfe < 2 || cfg.nfe > 64 || cfg.vocab_size < 25 || cfg.audio_vocab < 9022 ||
      cfg.acoustic_levels < 2 || (cfg.kv_f16 != 0 && cfg.kv_f16 != 1) ||
      (cfg.codec != 0 && cfg.codec != 1))
    return fail(nullptr, VX_E_INVALID, "config out of range");
  if (max_seq < 1 || max_seq > (1 << 20))
    return fail(nullptr, VX_E_INVALID, "max_seq_len %d out of range", max_seq);
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev < 1)
    return fail(nullptr, VX_E_DEVICE, "No HIP device");

  vx_engine *e = new vx_engine();
  e->cfg = cfg;
  {
    const char *ng = getenv("VX_NO_GRAPH");
    e->use_graphs = !(ng && ng[0] && ng[0] != '0');
  }
  e->max_seq = max_seq;
  e->kv_f32 = cfg.kv_f16 ? 0 : 1;
  e->kv_elem = cfg.kv_f16 ? 2 : 4;
  if (hipStreamCreateWithFlags(&e->st, hipStreamNonBlocking) != hipSuccess) {
    delete e;
    return fail(nullptr, VX_E_DEVICE, "hipStreamCreate failed");
  }
  // the decode attention partials take 35 KB (f16 cache) or 67 KB (f32)
  // of dynamic LDS for their two tile stages
  if (hipFuncSetAttribute((const void *)attn_partial_kernel<float>, hipFuncAttributeMaxDynamicSharedMemorySize,
                          KvRing<float>::LDS) != hipSuccess ||
      hipFuncSetAttribute((const void *)attn_partial_kernel<uint16_t>, hipFuncAttributeMaxDynamicSharedMemorySize,
                          KvRing<uint16_t>::LDS) != hipSuccess) {
    vx_destroy(e);
    return fail(nullptr, VX_E_DEVICE, "attention LDS attribute rejected");
  }
  (void)hipEventCreate(&e->ev0);
  (void)hipEventCreate(&e->ev1);
  (void)hipEventCreateWithFlags(&e->ev_frame[0], hipEventDisableTiming);
  (void)hipEventCreateWithFlags(&e->ev_frame[1], hipEventDisableTiming);
  // coherent (uncached) pinned memory: the frame's codes are stored into it
  // by fm_finish_kernel / topp_sample_kernel, visible to the host once the
  // frame's event has completed
  if (hipHostMalloc((void **)&e->h_frame, 2 * (1 + NAC) * 4, hipHostMallocMapped | hipHostMallocCoherent) !=
          hipSuccess ||
      hipHostGetDevicePointer((void **)&e->d_frame, e->h_frame, 0) != hipSuccess) {
    vx_destroy(e);
    return fail(nullptr, VX_E_NOMEM, "hipHostMalloc of readback slots failed");
  }

  // ---- weight table (names: src/engine.ts:659-743)
  struct Req {
    std::string name;
    std::vector<int64_t> shape;
    bool norm;
    uint16_t **dst;
    size_t off_rows;  // for q/k/v inside the stacked QKV matrix
  };
  const int nl = cfg.n_layers, fl = cfg.fm_layers;
  e->L.resize(nl);
  e->FL.resize(fl);
  size_t total = 0;
  auto reserve = [&](size_t elems) {
    size_t o = total;
    total += align256(elems * 2);
    return o;
  };
  // offsets first, pointers after the arena exists
  struct Off {
    uint16_t **dst;
    size_t off;
  };
  std::vector<Off> offs;
  auto place = [&](uint16_t **dst, size_t elems) { offs.push_back({dst, reserve(elems)}); };
  place(&e->tok_emb, (size_t)cfg.vocab_size * DIM);
  place(&e->audio_emb, (size_t)cfg.audio_vocab * DIM);
  place(&e->final_norm, DIM);
  auto place_layer = [&](LayerW &W) {
    place(&W.wqkv, (size_t)QKV_ROWS * DIM);
    place(&W.wo, (size_t)DIM * QD);
    place(&W.w1, (size_t)HID * DIM);
    place(&W.w3, (size_t)HID * DIM);
    place(&W.w2, (size_t)DIM * HID);
    place(&W.attn_norm, DIM);
    place(&W.ffn_norm, DIM);
  };
  for (auto &W : e->L) place_layer(W);
  for (auto &W : e->FL) place_layer(W);
  place(&e->fm_in, (size_t)DIM * NAC);
  place(&e->fm_time, (size_t)DIM * DIM);
  place(&e->fm_norm, DIM);
  // llm_projection and the semantic head are adjacent: both read W.normed,
  // so one GEMV streams the 3072 + 8320 rows (their outputs are adjacent too)
  place(&e->fm_llm, (size_t)DIM * DIM);
  place(&e->fm_sem, (size_t)SEMV * DIM);
  place(&e->fm_ac, (size_t)NAC * DIM);
  e->codec_on = cfg.codec != 0;
  CodecW &cw = e->cw;
  if (e->codec_on) {
    place(&cw.in_w, (size_t)CD * CIN * CK_IN);
    place(&cw.in_g, CD);
    for (int st = 0; st < CX_STAGES; st++) {
      for (auto &L : cw.L[st]) {
        place(&L.wqkv, (size_t)3 * CD * CD);
        place(&L.wo, (size_t)CD * CD);
        place(&L.w13, (size_t)2 * CHID * CD);
        place(&L.w2, (size_t)CD * CHID);
        place(&L.attn_norm, CD);
        place(&L.q_norm, CD);
        place(&L.k_norm, CD);
        place(&L.attn_scale, CD);
        place(&L.ffn_norm, CD);
        place(&L.ffn_scale, CD);
      }
      if (st < CX_STAGES - 1) {
        place(&cw.up_w[st], (size_t)CD * CD * CK_UP);
        place(&cw.up_g[st], CD);
      }
    }
    place(&cw.out_w, (size_t)CPATCH * CD * CK_OUT);
    place(&cw.out_g, CPATCH);
    place(&cw.cb_sum, (size_t)CSEM * CSEMD);
    place(&cw.cb_usage, CSEM);
  }
  if (hipMalloc(&e->warena, total) != hipSuccess) {
    vx_destroy(e);
    return fail(nullptr, VX_E_NOMEM, "hipMalloc of %zu weight bytes failed", total);
  }
  for (auto &o : offs) *o.dst = (uint16_t *)((char *)e->warena + o.off);
  if (e->fm_sem != e->fm_llm + (size_t)DIM * DIM) {  // one GEMV streams both (enqueue_fm)
    vx_destroy(e);
    return fail(nullptr, VX_E_STATE, "llm_projection and the semantic head are not adjacent");
  }

  add_slot(e, "mm_audio_embeddings.tok_embeddings.weight", e->tok_emb, {cfg.vocab_size, DIM}, false);
  add_slot(e, "mm_audio_embeddings.audio_codebook_embeddings.embeddings.weight", e->audio_emb,
           {cfg.audio_vocab, DIM}, false);
  add_slot(e, "norm.weight", e->final_norm, {DIM}, true);
  auto layer_slots = [&](const std::string &p, LayerW &W) {
    add_slot(e, p + ".attention_norm.weight", W.attn_norm, {DIM}, true);
    add_slot(e, p + ".attention.wq.weight", W.wqkv, {QD, DIM}, false);
    add_slot(e, p + ".attention.wk.weight", W.wqkv + (size_t)QD * DIM, {KVD, DIM}, false);
    add_slot(e, p + ".attention.wv.weight", W.wqkv + (size_t)(QD + KVD) * DIM, {KVD, DIM}, false);
    add_slot(e, p + ".attention.wo.weight", W.wo, {DIM, QD}, false);
    add_slot(e, p + ".ffn_norm.weight", W.ffn_norm, {DIM}, true);
    add_slot(e, p + ".feed_forward.w1.weight", W.w1, {HID, DIM}, false);
    add_slot(e, p + ".feed_forward.w2.weight", W.w2, {DIM, HID}, false);
    add_slot(e, p + ".feed_forward.w3.weight", W.w3, {HID, DIM}, false);
  };
  for (int i = 0; i < nl; i++) layer_slots("layers." + std::to_string(i), e->L[i]);
  for (int i = 0; i < fl; i++)
    layer_slots("acoustic_transformer.layers." + std::to_string(i), e->FL[i]);
  add_slot(e, "acoustic_transformer.input_projection.weight", e->fm_in, {DIM, NAC}, false);
  add_slot(e, "acoustic_transformer.llm_projection.weight", e->fm_llm, {DIM, DIM}, false);
  add_slot(e, "acoustic_transformer.time_projection.weight", e->fm_time, {DIM, DIM}, false);
  add_slot(e, "acoustic_transformer.norm.weight", e->fm_norm, {DIM}, true);
  add_slot(e, "acoustic_transformer.semantic_codebook_output.weight", e->fm_sem, {SEMV, DIM}, false);
  add_slot(e, "acoustic_transformer.acoustic_codebook_output.weight", e->fm_ac, {NAC, DIM}, false);
  if (e->codec_on) {
    // codec decoder tensors (src/engine.ts:700-770); weight-norm convs keep
    // v (original1) and g (original0) as stored
    const std::string P = "audio_tokenizer.";
    const int64_t cd = CD, hid = CHID;
    add_slot(e, P + "decoder_blocks.0.conv.parametrizations.weight.original1", cw.in_w,
             {cd, CIN, CK_IN}, false);
    add_slot(e, P + "decoder_blocks.0.conv.parametrizations.weight.original0", cw.in_g, {cd, 1, 1},
             true);
    for (int st = 0; st < CX_STAGES; st++) {
      for (int l = 0; l < CX_LPS; l++) {
        const CodecLayerW &L = cw.L[st][l];
        const std::string p =
            P + "decoder_blocks." + std::to_string(1 + 2 * st) + ".layers." + std::to_string(l) + ".";
        add_slot(e, p + "attention_norm.weight", L.attn_norm, {cd}, true);
        add_slot(e, p + "attention.q_norm.weight", L.q_norm, {cd}, true);
        add_slot(e, p + "attention.k_norm.weight", L.k_norm, {cd}, true);
        add_slot(e, p + "attention.wq.weight", L.wqkv, {cd, cd}, false);
        add_slot(e, p + "attention.wk.weight", L.wqkv + (size_t)CD * CD, {cd, cd}, false);
        add_slot(e, p + "attention.wv.weight", L.wqkv + (size_t)2 * CD * CD, {cd, cd}, false);
        add_slot(e, p + "attention.wo.weight", L.wo, {cd, cd}, false);
        add_slot(e, p + "attention_scale", L.attn_scale, {cd}, true);
        add_slot(e, p + "ffn_norm.weight", L.ffn_norm, {cd}, true);
        add_slot(e, p + "feed_forward.w1.weight", L.w13, {hid, cd}, false);
        add_slot(e, p + "feed_forward.w3.weight", L.w13 + (size_t)CHID * CD, {hid, cd}, false);
        add_slot(e, p + "feed_forward.w2.weight", L.w2, {cd, hid}, false);
        add_slot(e, p + "ffn_scale", L.ffn_scale, {cd}, true);
      }
      if (st < CX_STAGES - 1) {
        const std::string b =
            P + "decoder_blocks." + std::to_string(2 + 2 * st) + ".conv.parametrizations.weight.";
        add_slot(e, b + "original1", cw.up_w[st], {cd, cd, CK_UP}, false);
        add_slot(e, b + "original0", cw.up_g[st], {cd, 1, 1}, true);
      }
    }
    add_slot(e, P + "output_proj.conv.parametrizations.weight.original1", cw.out_w,
             {CPATCH, cd, CK_OUT}, false);
    add_slot(e, P + "output_proj.conv.parametrizations.weight.original0", cw.out_g, {CPATCH, 1, 1},
             true);
    add_slot(e, P + "quantizer.semantic_codebook.embedding_sum", cw.cb_sum, {CSEM, CSEMD}, false);
    add_slot(e, P + "quantizer.semantic_codebook.cluster_usage", cw.cb_usage, {CSEM}, true);

    // derived operands
    std::vector<std::pair<void **, size_t>> parts = {
        {(void **)&e->cx_cb, (size_t)CSEM * CSEMD * 2},
        {(void **)&e->cx_ain, (size_t)CD * CKIN * 2},
        {(void **)&e->cx_aout, (size_t)CPATCH_ROWS * CKOUT * 2},
        {(void **)&e->cx_rs_in, (size_t)CD * 4},
        {(void **)&e->cx_rs_out, (size_t)CPATCH_ROWS * 4}};
    for (int st = 0; st < CX_STAGES - 1; st++) {
      parts.push_back({(void **)&e->cx_aup[st], (size_t)2 * CD * CKUP * 2});
      parts.push_back({(void **)&e->cx_s_up[st], (size_t)CD * 4});
    }
    size_t tot = 0;
    for (auto &q : parts) tot += align256(q.second);
    if (hipMalloc(&e->cx_parena, tot) != hipSuccess) {
      vx_destroy(e);
      return fail(nullptr, VX_E_NOMEM, "hipMalloc of %zu codec operand bytes failed", tot);
    }
    char *p = (char *)e->cx_parena;
    for (auto &q : parts) {
      *q.first = p;
      p += align256(q.second);
    }
    if (const char *ch = getenv("VX_CODEC_CHUNK")) {  // tokens per codec GEMM (tuning, tests)
      const int v = atoi(ch);
      if (v >= 128 && v <= CX_MAXT && v % 128 == 0) e->cx_chunk = v;
    }
  }

  // ---- batched prefill buffers (one chunk of PF_MAXT tokens)
  if (const char *ch = getenv("VX_PREFILL_CHUNK")) {  // tokens per prefill chunk (tuning, tests)
    const int v = atoi(ch);
    if (v >= 128 && v <= PF_MAXT && v % 128 == 0) e->pf_chunk = v;
  }
  {
    std::vector<std::pair<void **, size_t>> parts = {
        {(void **)&e->pf_x, (size_t)PF_MAXT * DIM * 4},
        {(void **)&e->pf_q, (size_t)PF_MAXT * QD * 4},
        {(void **)&e->pf_c, (size_t)PF_NC * 2 * HID * 4},
        {(void **)&e->pf_b, (size_t)HID / 8 * PF_NC * 16},
        {(void **)&e->pf_voice, (size_t)PF_MAXT * DIM * 4},
        {(void **)&e->pf_tok, (size_t)PF_MAXT * 4}};
    size_t tot = 0;
    for (auto &q : parts) tot += align256(q.second);
    if (hipMalloc(&e->pf_arena, tot) != hipSuccess) {
      vx_destroy(e);
      return fail(nullptr, VX_E_NOMEM, "hipMalloc of %zu prefill bytes failed", tot);
    }
    char *p = (char *)e->pf_arena;
    for (auto &q : parts) {
      *q.first = p;
      p += align256(q.second);
    }
  }

  // ---- FM layer matrices in MFMA operand order
  {
    const size_t per = align256((size_t)QKV_ROWS * DIM * 2) + align256((size_t)DIM * QD * 2) +
                       2 * align256((size_t)HID * DIM * 2) + align256((size_t)DIM * HID * 2);
    if (hipMalloc(&e->fm_parena, per * fl) != hipSuccess) {
      vx_destroy(e);
      return fail(nullptr, VX_E_NOMEM, "hipMalloc of %zu packed FM weight bytes failed", per * fl);
    }
    e->FP.resize(fl);
    char *p = (char *)e->fm_parena;
    auto take = [&](uint16_t **dst, size_t elems) {
      *dst = (uint16_t *)p;
      p += align256(elems * 2);
    };
    for (auto &P : e->FP) {
      take(&P.wqkv, (size_t)QKV_ROWS * DIM);
      take(&P.wo, (size_t)DIM * QD);
      take(&P.w1, (size_t)HID * DIM);
      take(&P.w3, (size_t)HID * DIM);
      take(&P.w2, (size_t)DIM * HID);
    }
  }

  // ---- KV cache
  size_t kvbytes = (size_t)nl * 2 * NKV * max_seq * HD * e->kv_elem;
  if (hipMalloc(&e->kv, kvbytes) != hipSuccess) {
    vx_destroy(e);
    return fail(nullptr, VX_E_NOMEM, "hipMalloc of %zu KV bytes failed", kvbytes);
  }
  (void)hipMemsetAsync(e->kv, 0, kvbytes, e->st);

  // ---- activations
  size_t abytes = 0;
  std::vector<std::pair<void **, size_t>> aoffs;
  auto aplace = [&](void **dst, size_t bytes) {
    aoffs.push_back({dst, abytes});
    abytes += align256(bytes);
  };
  const int ns = cfg.nfe - 1;
  aplace((void **)&e->x, DIM * 4);
  aplace((void **)&e->q, QD * 4);
  aplace((void **)&e->attn, QD * 4);
  aplace((void **)&e->act, HID * 4);
  aplace((void **)&e->normed, DIM * 4);
  aplace((void **)&e->logits, (size_t)cfg.vocab_size * 4);
  aplace((void **)&e->part, (size_t)NH * ATTN_SPLITS * (HD + 2) * 4);
  aplace((void **)&e->layer_stage, (size_t)(nl * 4 + 1) * DIM * 4);
  aplace((void **)&e->pos, 4);
  aplace((void **)&e->frame, 4);
  aplace((void **)&e->sem_code, 4);
  aplace((void **)&e->codes, 64 * 4);
  aplace((void **)&e->argmax_res, 4);
  aplace((void **)&e->noise_seed, 8);
  aplace((void **)&e->rng_state, 8);
  aplace((void **)&e->tp_params, 16);
  aplace((void **)&e->tp_logits, (size_t)TP_MAXN * 4);
  aplace((void **)&e->fm_seq, 6 * DIM * 4);
  aplace((void **)&e->fm_q, 6 * QD * 4);
  aplace((void **)&e->fm_k, 6 * KVD * 4);
  aplace((void **)&e->fm_v, 6 * KVD * 4);
  aplace((void **)&e->fm_attn, 6 * QD * 4);
  aplace((void **)&e->fm_act, 6 * HID * 4);
  aplace((void **)&e->fm_llm_out, DIM * 4);
  aplace((void **)&e->sem_logits, SEMV * 4);
  aplace((void **)&e->timeline, (size_t)(6 * cfg.n_layers + 1) * TS_BLOCKS * 16);
  aplace((void **)&e->x_prev, DIM * 4);
  aplace((void **)&e->normed_prev, DIM * 4);
  aplace((void **)&e->logits_prev, SEMV * 4);
  aplace((void **)&e->tproj, (size_t)ns * DIM * 4);
  aplace((void **)&e->xh, (size_t)(ns + 1) * NAC * 4);
  aplace((void **)&e->vel, (size_t)ns * 2 * NAC * 4);
  aplace((void **)&e->ac_part, (size_t)2 * NAC * SSQ_MAX * 4);
  aplace((void **)&e->ac_ssq, (size_t)2 * SSQ_MAX * 4);
  aplace((void **)&e->noise, NAC * 4);
  aplace((void **)&e->time_embed, DIM * 4);
  aplace((void **)&e->inv_freq, HD / 2 * 4);
  aplace((void **)&e->fm_b_attn, (size_t)DIM / 8 * BCOL * 16);
  aplace((void **)&e->fm_b_o, (size_t)QD / 8 * BCOL * 16);
  aplace((void **)&e->fm_b_ffn, (size_t)DIM / 8 * BCOL * 16);
  aplace((void **)&e->fm_b_act, (size_t)HID / 8 * BCOL * 16);
  aplace((void **)&e->fm_ssq_attn, (size_t)SSQ_MAX * FMV * 4);
  aplace((void **)&e->fm_ssq_ffn, (size_t)SSQ_MAX * FMV * 4);
  if (hipMalloc(&e->aarena, abytes) != hipSuccess) {
    vx_destroy(e);
    return fail(nullptr, VX_E_NOMEM, "hipMalloc of activations failed");
  }
  for (auto &o : aoffs) *o.first = (char *)e->aarena + o.second;
  if (e->sem_logits != e->fm_llm_out + DIM) {  // written by one GEMV (enqueue_fm)
    vx_destroy(e);
    return fail(nullptr, VX_E_STATE, "fm_hidden and the semantic logits are not adjacent");
  }
  (void)hipMemsetAsync(e->aarena, 0, abytes, e->st);
  // rope frequencies, src/shaders.ts:224-256: freq_i = 1 / theta^(2i/128), evaluated once
  // here in f32 (the shader evaluates the same expression per element)
  float inv_freq[HD / 2];
  for (int i = 0; i < HD / 2; i++)
    inv_freq[i] = 1.0f / powf(cfg.rope_theta, (float)(i * 2) / (float)HD);
  (void)hipMemcpyAsync(e->inv_freq, inv_freq, sizeof inv_freq, hipMemcpyHostToDevice, e->st);
  if (hipStreamSynchronize(e->st) != hipSuccess) {
    vx_destroy(e);
    return fail(nullptr, VX_E_DEVICE, "device initialisation failed");
  }

  *out = e;
  return VX_OK;
}

void vx_destroy(vx_engine *e) {
  if (!e) return;
  if (e->st) (void)hipStreamSynchronize(e->st);
  if (e->step_exec) (void)hipGraphExecDestroy(e->step_exec);
  if (e->hold_exec) (void)hipGraphExecDestroy(e->hold_exec);
  if (e->timeline_exec) (void)hipGraphExecDestroy(e->timeline_exec);
  if (e->feedback_exec) (void)hipGraphExecDestroy(e->feedback_exec);
  if (e->fm_greedy_exec) (void)hipGraphExecDestroy(e->fm_greedy_exec);
  if (e->fm_topp_exec) (void)hipGraphExecDestroy(e->fm_topp_exec);
  if (e->frame_topp_exec) (void)hipGraphExecDestroy(e->frame_topp_exec);
  for (auto &ev : e->ev_frame)
    if (ev) (void)hipEventDestroy(ev);
  if (e->h_frame) (void)hipHostFree(e->h_frame);
  if (e->fm_plain_exec) (void)hipGraphExecDestroy(e->fm_plain_exec);
  if (e->frame_exec) (void)hipGraphExecDestroy(e->frame_exec);
  if (e->warena) (void)hipFree(e->warena);
  if (e->kv) (void)hipFree(e->kv);
  if (e->fm_parena) (void)hipFree(e->fm_parena);
  if (e->pf_arena) (void)hipFree(e->pf_arena);
  if (e->cx_parena) (void)hipFree(e->cx_parena);
  if (e->cx_arena) (void)hipFree(e->cx_arena);
  if (e->aarena) (void)hipFree(e->aarena);
  if (e->ev0) (void)hipEventDestroy(e->ev0);
  if (e->ev1) (void)hipEventDestroy(e->ev1);
  if (e->st) (void)hipStreamDestroy(e->st);
  delete e;
}

int vx_load_tensor(vx_engine *e, const char *name, const uint16_t *f16, size_t numel,
                   const int64_t *shape, int32_t ndim) {
  if (!e || !name || !f16) return e ? fail(e, VX_E_INVALID, "NULL argument") : VX_E_INVALID;
  auto it = e->slots.find(name);
  if (it == e->slots.end()) return fail(e, VX_E_INVALID, "Unknown tensor: %s", name);
  Slot &s = it->second;
  if (numel != s.numel) return fail(e, VX_E_INVALID, "%s: %zu elements, expected %zu", name, numel, s.numel);
  if (shape) {
    if ((size_t)ndim != s.shape.size())
      return fail(e, VX_E_INVALID, "%s: rank %d, expected %zu", name, ndim, s.shape.size());
    for (int i = 0; i < ndim; i++)
      if (shape[i] != s.shape[i]) return fail(e, VX_E_INVALID, "%s: shape mismatch in dim %d", name, i);
  }
  HIPCHK(e, hipMemcpyAsync(s.ptr, f16, numel * 2, hipMemcpyHostToDevice, e->st));
  HIPCHK(e, hipStreamSynchronize(e->st));
  s.loaded = true;
  if (s.ptr == e->fm_time) e->tproj_ready = false;
  e->fm_packed_ready = false;
  e->codec_ready = false;
  return VX_OK;
}

// ------------------------------------------------------------ safetensors
void vx_bf16_to_f16(const uint16_t *in, uint16_t *out, size_t n) {
  for (size_t i = 0; in && out && i < n; i++) out[i] = bf16_to_f16_ref(in[i]);
}
void vx_f32_to_f16_trunc(const float *in, uint16_t *out, size_t n) {
  for (size_t i = 0; in && out && i < n; i++) {
    uint32_t b;
    memcpy(&b, in + i, 4);
    out[i] = f32_to_f16_ref(b);
  }
}

int vx_load_safetensors(vx_engine *e, const char *path, int32_t *n_loaded, int32_t *n_skipped) {
  return vx_load_safetensors_progress(e, path, nullptr, nullptr, n_loaded, n_skipped);
}

int vx_missing_tensor(const vx_engine *e, char *name, int32_t cap) {
  if (!e) return 0;
  for (auto &kv : e->slots)
    if (!kv.second.loaded) {
      if (name && cap > 0) snprintf(name, (size_t)cap, "%s", kv.first.c_str());
      return 1;
    }
  return 0;
}

int vx_load_safetensors_progress(vx_engine *e, const char *path, vx_load_cb on_tensor, void *user,
                                 int32_t *n_loaded, int32_t *n_skipped) {
  if (!e || !path) return VX_E_INVALID;
  const int fd = open(path, O_RDONLY);
  if (fd < 0) return fail(e, VX_E_INVALID, "cannot open %s", path);
  struct FdGuard {
    int fd;
    ~FdGuard() { close(fd); }
  } guard{fd};
  const off_t fsize = lseek(fd, 0, SEEK_END);
  uint64_t hlen = 0;
  if (fsize < 8 || pread(fd, &hlen, 8, 0) != 8 || hlen == 0 || hlen > (uint64_t)fsize - 8 ||
      hlen > (64ull << 20))
    return fail(e, VX_E_INVALID, "%s: not a safetensors file", path);
  std::string hdr(hlen, '\0');
  if (pread(fd, &hdr[0], hlen, 8) != (ssize_t)hlen)
    return fail(e, VX_E_INVALID, "%s: short read of the header", path);
  std::map<std::string, StEntry> entries;
  std::string perr;
  if (!StHeaderParser(hdr.data(), hdr.size()).parse(entries, perr))
    return fail(e, VX_E_INVALID, "%s: bad safetensors header: %s", path, perr.c_str());
  const uint64_t data0 = 8 + hlen;
  // validate every tensor the engine takes before touching the device
  std::vector<std::pair<const std::string *, Slot *>> work;
  int skipped = 0;
  for (auto &kv : entries) {
    auto it = e->slots.find(kv.first);
    if (!strcmp(st_component(kv.first), "other") || it == e->slots.end()) {
      skipped++;  // names the engine does not use (codec tensors when it has no codec)
      continue;
    }
    const StEntry &t = kv.second;
    const std::string &dt = t.dtype;
    if (dt != "BF16" && dt != "F16" && dt != "F32")  // src/weights.ts:590-592
      return fail(e, VX_E_INVALID, "Unsupported dtype for %s: %s", kv.first.c_str(), dt.c_str());
    const uint64_t es = dt == "F32" ? 4 : 2;
    Slot &sl = it->second;
    if ((t.end - t.begin) != sl.numel * es || data0 + t.end > (uint64_t)fsize)
      return fail(e, VX_E_INVALID, "%s: %llu bytes, expected %zu", kv.first.c_str(),
                  (unsigned long long)(t.end - t.begin), sl.numel * es);
    if (t.shape != sl.shape) return fail(e, VX_E_INVALID, "%s: shape mismatch", kv.first.c_str());
    work.push_back({&kv.first, &sl});
  }
  // component order backbone, fm, codec (src/weights.ts:520-523); names in
  // order within a component
  auto rank = [](const std::string &n) {
    const char *c = st_component(n);
    return !strcmp(c, "backbone") ? 0 : !strcmp(c, "fm") ? 1 : 2;
  };
  std::stable_sort(work.begin(), work.end(),
                   [&](const auto &a, const auto &b) { return rank(*a.first) < rank(*b.first); });
  uint64_t bytes_read = 8 + hlen;
  int32_t done_tensors = 0;
  // stream each tensor through a device staging buffer; convert on the GPU
  constexpr size_t CH = 256u << 20;
  void *stage = nullptr;
  std::vector<char> host(CH);
  HIPCHK(e, hipMalloc(&stage, CH));
  struct DevGuard {
    void *p;
    ~DevGuard() { (void)hipFree(p); }
  } dguard{stage};
  for (auto &w : work) {
    const StEntry &t = entries[*w.first];
    const bool f32 = t.dtype == "F32", bf16 = t.dtype == "BF16";
    const size_t es = f32 ? 4 : 2;
    for (size_t done = 0; done < t.end - t.begin;) {
      const size_t len = std::min(CH, (size_t)(t.end - t.begin) - done);
      if (pread(fd, host.data(), len, (off_t)(data0 + t.begin + done)) != (ssize_t)len)
        return fail(e, VX_E_INVALID, "%s: short read of %s", path, w.first->c_str());
      uint16_t *dst = w.second->ptr + done / es;
      if (!f32 && !bf16) {
        HIPCHK(e, hipMemcpy(dst, host.data(), len, hipMemcpyHostToDevice));
      } else {
        HIPCHK(e, hipMemcpy(stage, host.data(), len, hipMemcpyHostToDevice));
        if (bf16)
          hipLaunchKernelGGL(bf16_to_f16_kernel, dim3(2048), dim3(256), 0, e->st, (const uint16_t *)stage,
                             dst, len / 2);
        else
          hipLaunchKernelGGL(f32_to_f16_ref_kernel, dim3(2048), dim3(256), 0, e->st,
                             (const uint32_t *)stage, dst, len / 4);
        LAUNCHCHK(e);
        HIPCHK(e, hipStreamSynchronize(e->st));
      }
      done += len;
      bytes_read += len;
    }
    w.second->loaded = true;
    done_tensors++;
    if (on_tensor)
      on_tensor(user, done_tensors, (int32_t)work.size(), st_component(*w.first), w.first->c_str(), bytes_read);
  }
  e->weights_changed();
  if (n_loaded) *n_loaded = (int32_t)work.size();
  if (n_skipped) *n_skipped = skipped;
  return VX_OK;
}

int vx_init_synthetic(vx_engine *e, uint64_t seed, float std) {
  if (!e) return VX_E_INVALID;
  for (auto &kv : e->slots) {
    Slot &s = kv.second;
    size_t blocks = std::min<size_t>((s.numel + 255) / 256, 65536);
    hipLaunchKernelGGL(gen_f16_kernel, dim3((unsigned)blocks), dim3(256), 0, e->st, s.ptr, s.numel,
                       seed, fnv1a(kv.first.c_str()), s.is_norm ? 1.0f : 0.0f, std);
    s.loaded = true;
  }
  LAUNCHCHK(e);
  HIPCHK(e, hipStreamSynchronize(e->st));
  e->weights_changed();
  return VX_OK;
}

int vx_read_tensor(vx_engine *e, const char *name, uint16_t *f16, size_t numel) {
  if (!e || !name || !f16) return e ? fail(e, VX_E_INVALID, "NULL argument") : VX_E_INVALID;
  auto it = e->slots.find(name);
  if (it == e->slots.end()) return fail(e, VX_E_INVALID, "Unknown tensor: %s", name);
  if (numel > it->second.numel)
    return fail(e, VX_E_INVALID, "%s holds %zu elements", name, it->second.numel);
  HIPCHK(e, hipMemcpyAsync(f16, it->second.ptr, numel * 2, hipMemcpyDeviceToHost, e->st));
  HIPCHK(e, hipStreamSynchronize(e->st));
  return VX_OK;
}

int vx_is_ready(const vx_engine *e) {
  if (!e) return 0;
  for (auto &kv : e->slots)
    if (!kv.second.loaded) return 0;
  return 1;
}

int vx_set_position(vx_engine *e, int32_t p) {
  if (!e) return VX_E_INVALID;
  if (p < 0 || p > e->max_seq) return fail(e, VX_E_RANGE, "position %d out of range", p);
  hipLaunchKernelGGL(set_int_kernel, dim3(1), dim3(1), 0, e->st, e->pos, p);
  LAUNCHCHK(e);
  e->host_pos = p;
  return VX_OK;
}

int vx_reset(vx_engine *e) {
  if (!e) return VX_E_INVALID;
  hipLaunchKernelGGL(set_int_kernel, dim3(1), dim3(1), 0, e->st, e->frame, 0);
  return vx_set_position(e, 0);
}

int32_t vx_position(const vx_engine *e) { return e ? e->host_pos : -1; }

int vx_synchronize(vx_engine *e) {
  if (!e) return VX_E_INVALID;
  HIPCHK(e, hipStreamSynchronize(e->st));
  return VX_OK;
}

int vx_backbone_step(vx_engine *e, int32_t token, int32_t mode, const float *pre, int32_t lm_head,
                     uint32_t *argmax_out, float *normed_out) {
  if (!e) return VX_E_INVALID;
  int rc = check_ready(e);
  if (rc) return rc;
  if ((rc = prepare_input(e, token, mode, pre))) return rc;
  if ((rc = run_step(e))) return rc;
  e->host_pos++;
  if (lm_head) {
    enqueue_lm_head(e);
    LAUNCHCHK(e);
  }
  if (argmax_out && lm_head)
    HIPCHK(e, hipMemcpyAsync(argmax_out, e->argmax_res, 4, hipMemcpyDeviceToHost, e->st));
  if (normed_out)
    HIPCHK(e, hipMemcpyAsync(normed_out, e->normed, DIM * 4, hipMemcpyDeviceToHost, e->st));
  HIPCHK(e, hipStreamSynchronize(e->st));
  return VX_OK;
}

// One eager step that stages the reference's per-layer read points
// (src/engine.ts:2106-2287) in layer_stage: the embedding (the first
// layer's input) in row 0, then per layer attn_norm, attn_out, ffn_norm,
// ffn_out.  The GEMVs fuse their RMSNorm, so the two norm outputs are
// formed here by the final-norm kernel with the layer's gains: the fused
// prologue's formula x * (1 / sqrt(sum x^2 / dim + eps)) * w, its sum of
// squares added in another order.
static int debug_layers_step(vx_engine *e, int32_t token, int32_t mode, const float *pre) {
  int rc = check_ready(e);
  if (rc) return rc;
  if ((rc = prepare_input(e, token, mode, pre))) return rc;
  const float eps = e->cfg.norm_eps;
  auto stage = [&](int row) { return e->layer_stage + (size_t)row * DIM; };
  HIPCHK(e, hipMemcpyAsync(stage(0), e->x, DIM * 4, hipMemcpyDeviceToDevice, e->st));
  for (int l = 0; l < e->cfg.n_layers; l++) {
    const int r = 1 + 4 * l;
    hipLaunchKernelGGL(final_norm_kernel, dim3(1), dim3(1024), 0, e->st, e->x, e->L[l].attn_norm, eps,
                       stage(r), nullptr, nullptr);
    enqueue_layer(e, l, VX_KERNEL_QKV);
    enqueue_layer(e, l, VX_KERNEL_ATTN);
    enqueue_layer(e, l, VX_KERNEL_OPROJ);
    HIPCHK(e, hipMemcpyAsync(stage(r + 1), e->x, DIM * 4, hipMemcpyDeviceToDevice, e->st));
    hipLaunchKernelGGL(final_norm_kernel, dim3(1), dim3(1024), 0, e->st, e->x, e->L[l].ffn_norm, eps,
                       stage(r + 2), nullptr, nullptr);
    enqueue_layer(e, l, VX_KERNEL_GATEUP);
    enqueue_layer(e, l, VX_KERNEL_DOWN);
    HIPCHK(e, hipMemcpyAsync(stage(r + 3), e->x, DIM * 4, hipMemcpyDeviceToDevice, e->st));
  }
  hipLaunchKernelGGL(final_norm_kernel, dim3(1), dim3(1024), 0, e->st, e->x, e->final_norm, eps, e->normed,
                     e->pos, nullptr);
  LAUNCHCHK(e);
  e->host_pos++;
  return VX_OK;
}

int vx_backbone_step_layers(vx_engine *e, int32_t token, int32_t mode, const float *pre,
                            float *layer_out) {
  if (!e || !layer_out) return VX_E_INVALID;
  int rc = debug_layers_step(e, token, mode, pre);
  if (rc) return rc;
  for (int l = 0; l < e->cfg.n_layers; l++)
    for (int k = 0; k < 2; k++)
      HIPCHK(e, hipMemcpyAsync(layer_out + (size_t)(2 * l + k) * DIM,
                               e->layer_stage + (size_t)(2 + 4 * l + 2 * k) * DIM, DIM * 4,
                               hipMemcpyDeviceToHost, e->st));
  HIPCHK(e, hipStreamSynchronize(e->st));
  return VX_OK;
}

int vx_debug_backbone_layers(vx_engine *e, int32_t token, int32_t mode, const float *pre, float *embed,
                             float *layers) {
  if (!e || (!embed && !layers)) return VX_E_INVALID;
  int rc = debug_layers_step(e, token, mode, pre);
  if (rc) return rc;
  if (embed) HIPCHK(e, hipMemcpyAsync(embed, e->layer_stage, DIM * 4, hipMemcpyDeviceToHost, e->st));
  if (layers)
    HIPCHK(e, hipMemcpyAsync(layers, e->layer_stage + DIM, (size_t)e->cfg.n_layers * 4 * DIM * 4,
                             hipMemcpyDeviceToHost, e->st));
  HIPCHK(e, hipStreamSynchronize(e->st));
  return VX_OK;
}

int vx_fm_forward(vx_engine *e, const float *noise, float *sem_logits, uint32_t *codes,
                  float *x_final) {
  if (!e) return VX_E_INVALID;
  int rc = check_ready(e);
  if (rc) return rc;
  if ((rc = ensure_tproj(e))) return rc;
  if (noise) HIPCHK(e, hipMemcpyAsync(e->noise, noise, NAC * 4, hipMemcpyHostToDevice, e->st));
  enqueue_fm(e, noise ? e->noise : nullptr, false);
  LAUNCHCHK(e);
  if (sem_logits)
    HIPCHK(e, hipMemcpyAsync(sem_logits, e->sem_logits, SEMV * 4, hipMemcpyDeviceToHost, e->st));
  if (codes) HIPCHK(e, hipMemcpyAsync(codes, e->codes, NAC * 4, hipMemcpyDeviceToHost, e->st));
  if (x_final)
    HIPCHK(e, hipMemcpyAsync(x_final, e->xh + (size_t)e->nsteps() * NAC, NAC * 4,
                             hipMemcpyDeviceToHost, e->st));
  HIPCHK(e, hipStreamSynchronize(e->st));
  return VX_OK;
}

int vx_set_semantic_code(vx_engine *e, uint32_t code) {
  if (!e) return VX_E_INVALID;
  // unsigned compare: a code of 2^31 or more must not pass as a negative int
  if (code >= (uint32_t)e->cfg.audio_vocab)
    return fail(e, VX_E_INVALID, "semantic code %u out of range", code);
  hipLaunchKernelGGL(set_u32_kernel, dim3(1), dim3(1), 0, e->st, e->sem_code, code);
  LAUNCHCHK(e);
  return VX_OK;
}

int vx_set_acoustic_codes(vx_engine *e, const uint32_t *c) {
  if (!e || !c) return VX_E_INVALID;
  for (int i = 0; i < NAC; i++)
    if (c[i] > 22) return fail(e, VX_E_INVALID, "acoustic code %u out of range", c[i]);
  HIPCHK(e, hipMemcpyAsync(e->codes, c, NAC * 4, hipMemcpyHostToDevice, e->st));
  HIPCHK(e, hipStreamSynchronize(e->st));
  return VX_OK;
}

int vx_get_codes(vx_engine *e, uint32_t *sem, uint32_t *c) {
  if (!e) return VX_E_INVALID;
  if (sem) HIPCHK(e, hipMemcpyAsync(sem, e->sem_code, 4, hipMemcpyDeviceToHost, e->st));
  if (c) HIPCHK(e, hipMemcpyAsync(c, e->codes, NAC * 4, hipMemcpyDeviceToHost, e->st));
  HIPCHK(e, hipStreamSynchronize(e->st));
  return VX_OK;
}

int vx_read(vx_engine *e, const char *name, float *dst, size_t count) {
  if (!e || !name || !dst) return VX_E_INVALID;
  struct B {
    const char *n;
    const float *p;
    size_t cnt;
  } t[] = {
      {"hidden", e->x, DIM},
      {"normed", e->normed, DIM},
      {"q", e->q, QD},
      {"attn_out", e->attn, QD},
      {"gate", e->act, HID},
      {"logits", e->logits, (size_t)e->cfg.vocab_size},
      {"semantic_logits", e->sem_logits, SEMV},
      {"x_t", e->xh + (size_t)e->nsteps() * NAC, NAC},
      {"velocity", e->vel + (size_t)(e->nsteps() - 1) * 2 * NAC, NAC},
      {"v_uncond", e->vel + (size_t)(e->nsteps() - 1) * 2 * NAC + NAC, NAC},
      {"fm_hidden", e->fm_llm_out, DIM},
      {"fm_seq", e->fm_seq, 6 * DIM},
      {"time_proj", e->tproj, (size_t)e->nsteps() * DIM},
      {"x_history", e->xh, (size_t)(e->nsteps() + 1) * NAC},
      {"velocity_history", e->vel, (size_t)e->nsteps() * 2 * NAC},
  };
  for (auto &b : t)
    if (!strcmp(b.n, name)) {
      if (count > b.cnt) return fail(e, VX_E_INVALID, "%s holds %zu values", name, b.cnt);
      HIPCHK(e, hipMemcpyAsync(dst, b.p, count * 4, hipMemcpyDeviceToHost, e->st));
      HIPCHK(e, hipStreamSynchronize(e->st));
      return VX_OK;
    }
  return fail(e, VX_E_INVALID, "Unknown buffer: %s", name);
}

int vx_write(vx_engine *e, const char *name, const float *src, size_t count) {
  if (!e || !name || !src) return VX_E_INVALID;
  float *dst = nullptr;
  if (!strcmp(name, "normed")) dst = e->normed;
  else if (!strcmp(name, "hidden")) dst = e->x;
  else return fail(e, VX_E_INVALID, "Unknown writable buffer: %s", name);
  if (count > (size_t)DIM) return fail(e, VX_E_INVALID, "%s holds %d values", name, DIM);
  HIPCHK(e, hipMemcpyAsync(dst, src, count * 4, hipMemcpyHostToDevice, e->st));
  HIPCHK(e, hipStreamSynchronize(e->st));
  return VX_OK;
}

static uint16_t host_f2h(float f) {  // IEEE round-to-nearest-even
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
  uint32_t q, rem, half;
  if (ax < 0x38800000u) {
    if (ax <= 0x33000000u) return (uint16_t)sign;
    const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    const int rsh = 126 - (int)(ax >> 23);
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
static float host_h2f(uint16_t h) {
  const uint32_t e = (h >> 10) & 31u, m = h & 0x3ffu;
  float v = e == 0 ? (float)m * 0x1p-24f
                   : e == 31 ? (m ? NAN : INFINITY) : std::ldexp((float)(m | 0x400u), (int)e - 25);
  return (h & 0x8000u) ? -v : v;
}

// caller layout [pos][kvh*128 + d] (f32) <-> device [kvh][pos][d] (f32 or f16)
static int kv_io(vx_engine *e, int32_t layer, int32_t which, int32_t pos0, int32_t npos,
                 float *host, bool write) {
  if (!e || !host) return VX_E_INVALID;
  if (layer < 0 || layer >= e->cfg.n_layers || which < 0 || which > 1 || pos0 < 0 || npos < 0 ||
      (int64_t)pos0 + npos > e->max_seq)
    return fail(e, VX_E_INVALID, "KV range out of bounds");
  if (npos == 0) return VX_OK;
  char *base = (char *)(which ? e->vc(layer) : e->kc(layer));
  const size_t es = e->kv_elem, n = (size_t)npos * KVD;
  std::vector<uint16_t> h16;
  void *hbuf = host;
  if (!e->kv_f32) {
    h16.resize(n);
    hbuf = h16.data();
    if (write)
      for (size_t i = 0; i < n; i++) h16[i] = host_f2h(host[i]);
  }
  for (int h = 0; h < NKV; h++) {
    char *dev = base + ((size_t)h * e->max_seq + pos0) * HD * es;
    char *hp = (char *)hbuf + (size_t)h * HD * es;
    if (write)
      HIPCHK(e, hipMemcpy2DAsync(dev, HD * es, hp, KVD * es, HD * es, npos, hipMemcpyHostToDevice,
                                 e->st));
    else
      HIPCHK(e, hipMemcpy2DAsync(hp, KVD * es, dev, HD * es, HD * es, npos, hipMemcpyDeviceToHost,
                                 e->st));
  }
  HIPCHK(e, hipStreamSynchronize(e->st));
  if (!e->kv_f32 && !write)
    for (size_t i = 0; i < n; i++) host[i] = host_h2f(h16[i]);
  return VX_OK;
}

int vx_write_kv(vx_engine *e, int32_t layer, int32_t which, int32_t pos0, int32_t npos,
                const float *src) {
  return kv_io(e, layer, which, pos0, npos, const_cast<float *>(src), true);
}

int vx_read_kv(vx_engine *e, int32_t layer, int32_t which, int32_t pos0, int32_t npos, float *dst) {
  return kv_io(e, layer, which, pos0, npos, dst, false);
}

int vx_fill_kv_synthetic(vx_engine *e, uint64_t seed, int32_t npos) {
  if (!e) return VX_E_INVALID;
  if (npos < 0 || npos > e->max_seq) return fail(e, VX_E_INVALID, "npos out of range");
  for (int l = 0; l < e->cfg.n_layers; l++)
    for (int w = 0; w < 2; w++) {
      std::string nm = "kv." + std::to_string(l) + (w ? ".v" : ".k");
      void *c = w ? e->vc(l) : e->kc(l);
      if (e->kv_f32)
        hipLaunchKernelGGL(gen_kv_kernel<float>, dim3(1024), dim3(256), 0, e->st, (float *)c,
                           e->max_seq, npos, seed, fnv1a(nm.c_str()));
      else
        hipLaunchKernelGGL(gen_kv_kernel<uint16_t>, dim3(1024), dim3(256), 0, e->st, (uint16_t *)c,
                           e->max_seq, npos, seed, fnv1a(nm.c_str()));
    }
  LAUNCHCHK(e);
  HIPCHK(e, hipStreamSynchronize(e->st));
  return VX_OK;
}

// -------------------------------------------------------------- prefill
// One chunk of n <= PF_MAXT prompt tokens (global indices tok0..tok0+n-1)
// through every layer at positions host_pos..host_pos+n-1; tokens and voice
// rows are already on the device.  Afterwards the residual stream and
// W.normed hold the last token's values and the position is advanced, as
// after n single steps.
// The prefill GEMMs (vx_gemm.h): 144 KB of dynamic LDS per block and the
// device's compute-unit count for the grids; the prompt attention's 71 KB.
static int pf_gemm_setup(vx_engine *e) {
  if (e->gemm_ready) return VX_OK;
  HIPCHK(e, gemm_setup());
  HIPCHK(e, hipFuncSetAttribute((const void *)pf_attn_mfma_kernel<float>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, PFA_LDS));
  HIPCHK(e, hipFuncSetAttribute((const void *)pf_attn_mfma_kernel<uint16_t>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, PFA_LDS));
  int dev = 0;
  HIPCHK(e, hipGetDevice(&dev));
  HIPCHK(e, hipDeviceGetAttribute(&e->cus, hipDeviceAttributeMultiprocessorCount, dev));
  if (e->cus < 8) return fail(e, VX_E_DEVICE, "unexpected compute unit count %d", e->cus);
  e->gemm_ready = true;
  return VX_OK;
}

// pf_c[s][col][m] for s < *ns: the ns K-slice partial sums of
// W[M][K] x pf_b (2 nt rows of K halves)
static int pf_gemm(vx_engine *e, const uint16_t *W, int M, int K, int nt, int *ns) {
  if (M % GM_BM || K % GM_BK || nt % GM_BN)
    return fail(e, VX_E_STATE, "prefill GEMM shape M %d K %d nt %d", M, K, nt);
  const GemmPlan p = gemm_plan(M, K, nt, e->cus);
  if (p.slices != 1 && p.slices != 2 && p.slices != 4 && p.slices != 8)
    return fail(e, VX_E_STATE, "prefill GEMM plan with %d slices", p.slices);
  if ((size_t)p.slices * nt * M > (size_t)PF_NC * 2 * HID)
    return fail(e, VX_E_STATE, "prefill GEMM output (%d slices of %d x %d) exceeds its buffer", p.slices, nt, M);
  gemm_launch(p, e->st, W, M, K, (const uint16_t *)e->pf_b, nt, e->pf_c);
  *ns = p.slices;
  return VX_OK;
}

// cx_c[s][col][m] for s < *ns: the codec chunk's K-slice partial sums of
// W[M][K] x cx_b (nc = 2 nt rows of K halves)
static int cx_gemm(vx_engine *e, const uint16_t *W, int M, int K, int nc, int *ns) {
  const int nt = nc / 2;
  if (M % GM_BM || K % GM_BK || nt % GM_BN)
    return fail(e, VX_E_STATE, "codec GEMM shape M %d K %d nt %d", M, K, nt);
  const GemmPlan p = gemm_plan(M, K, nt, e->cus);
  if (p.slices != 1 && p.slices != 2 && p.slices != 4 && p.slices != 8)
    return fail(e, VX_E_STATE, "codec GEMM plan with %d slices", p.slices);
  if ((size_t)p.slices * nt * M > CX_CCAP)
    return fail(e, VX_E_STATE, "codec GEMM output (%d slices of %d x %d) exceeds its buffer", p.slices, nt, M);
  gemm_launch(p, e->st, W, M, K, (const uint16_t *)e->cx_b, nt, e->cx_c);
  *ns = p.slices;
  return VX_OK;
}

static int enqueue_prefill_chunk(vx_engine *e, int n, int tok0, int vstart, int vcount,
                                 bool has_voice) {
  int rc = VX_OK, ns = 1;
  const int nt = pf_nt(n);
  hipStream_t st = e->st;
  const int pos0 = e->host_pos;
  hipLaunchKernelGGL(pf_embed_kernel, dim3(n, DIM / 256), dim3(256), 0, st, e->tok_emb, e->pf_tok,
                     has_voice ? e->pf_voice : nullptr, vstart, vcount, tok0, e->pf_x);
  const dim3 blk(256);
  // layer 0's B; every later B is written by the kernel producing its input
  hipLaunchKernelGGL(pf_pack_kernel<true>, dim3(nt), blk, 0, st, e->pf_x, DIM, n, nt,
                     e->L[0].attn_norm, e->cfg.norm_eps, e->pf_b);
  for (int l = 0; l < e->cfg.n_layers; l++) {
    const LayerW &W = e->L[l];
    const bool next = l + 1 < e->cfg.n_layers;
    if ((rc = pf_gemm(e, W.wqkv, QKV_ROWS, DIM, nt, &ns))) return rc;
    gm_with_slices(ns, [&](auto NS) {
      hipLaunchKernelGGL(pf_qkv_epi_kernel<NS>, dim3(n, QKV_ROWS / 2 / 256), blk, 0, st, e->pf_c, nt,
                         e->pf_q, e->kc(l), e->vc(l), e->kv_f32, e->max_seq, pos0, e->inv_freq);
    });
    if (e->kv_f32)
      hipLaunchKernelGGL(pf_attn_mfma_kernel<float>, dim3(nt / PFA_T, NKV), dim3(256 * PFA_KG), PFA_LDS,
                         st, e->pf_q, (const float *)e->kc(l), (const float *)e->vc(l), e->max_seq, pos0,
                         n, nt, e->pf_b);
    else
      hipLaunchKernelGGL(pf_attn_mfma_kernel<uint16_t>, dim3(nt / PFA_T, NKV), dim3(256 * PFA_KG),
                         PFA_LDS, st, e->pf_q, (const uint16_t *)e->kc(l), (const uint16_t *)e->vc(l),
                         e->max_seq, pos0, n, nt, e->pf_b);
    if ((rc = pf_gemm(e, W.wo, DIM, QD, nt, &ns))) return rc;
    gm_with_slices(ns, [&](auto NS) {
      hipLaunchKernelGGL((pf_resid_pack_kernel<true, NS>), dim3(nt), blk, 0, st, e->pf_c, n, nt, e->pf_x,
                         W.ffn_norm, e->cfg.norm_eps, e->pf_b);
    });
    // W1 and W3 are adjacent in the arena: one GEMM over the stacked rows
    if ((rc = pf_gemm(e, W.w1, 2 * HID, DIM, nt, &ns))) return rc;
    gm_with_slices(ns, [&](auto NS) {
      hipLaunchKernelGGL(pf_swiglu_pack_kernel<NS>, dim3(nt, HID / 8 / 128), dim3(128), 0, st, e->pf_c, n,
                         nt, e->pf_b);
    });
    if ((rc = pf_gemm(e, W.w2, DIM, HID, nt, &ns))) return rc;
    gm_with_slices(ns, [&](auto NS) {
      if (next)
        hipLaunchKernelGGL((pf_resid_pack_kernel<true, NS>), dim3(nt), blk, 0, st, e->pf_c, n, nt, e->pf_x,
                           e->L[l + 1].attn_norm, e->cfg.norm_eps, e->pf_b);
      else
        hipLaunchKernelGGL((pf_resid_pack_kernel<false, NS>), dim3(n), blk, 0, st, e->pf_c, n, nt, e->pf_x,
                           nullptr, 0.f, nullptr);
    });
  }
  (void)hipMemcpyAsync(e->x, e->pf_x + (size_t)(n - 1) * DIM, DIM * 4, hipMemcpyDeviceToDevice, st);
  hipLaunchKernelGGL(final_norm_kernel, dim3(1), dim3(1024), 0, st, e->x, e->final_norm,
                     e->cfg.norm_eps, e->normed, nullptr, nullptr);
  hipLaunchKernelGGL(set_int_kernel, dim3(1), dim3(1), 0, st, e->pos, pos0 + n);
  e->host_pos = pos0 + n;
  return VX_OK;
}

int vx_prefill(vx_engine *e, const int32_t *tokens, int32_t n_tokens, int32_t audio_start,
               int32_t audio_count, const float *voice) {
  if (!e) return VX_E_INVALID;
  int rc = check_ready(e);
  if (rc) return rc;
  if (n_tokens < 1 || !tokens || audio_count < 0 || (audio_count > 0 && audio_start < 0) ||
      (int64_t)audio_start + audio_count > INT32_MAX)
    return fail(e, VX_E_INVALID, "bad prefill arguments");
  if ((int64_t)e->host_pos + n_tokens > e->max_seq)
    return fail(e, VX_E_RANGE, "prefill passes max_seq_len %d", e->max_seq);
  for (int i = 0; i < n_tokens; i++)
    if (tokens[i] < 0 || tokens[i] >= e->cfg.vocab_size)
      return fail(e, VX_E_INVALID, "token %d out of range", tokens[i]);
  if (e->L[0].w3 != e->L[0].w1 + (size_t)HID * DIM)
    return fail(e, VX_E_STATE, "weight layout: gate and up matrices not adjacent");
  if ((rc = pf_gemm_setup(e))) return rc;
  const bool has_voice = voice && audio_count > 0;
  for (int c0 = 0; c0 < n_tokens; c0 += e->pf_chunk) {
    const int n = std::min(e->pf_chunk, n_tokens - c0);
    HIPCHK(e, hipMemcpyAsync(e->pf_tok, tokens + c0, (size_t)n * 4, hipMemcpyHostToDevice, e->st));
    // voice rows of this chunk, at chunk-local offsets
    int vs = 0, vc = 0;
    if (has_voice) {
      const int a = std::max(c0, audio_start), b = std::min(c0 + n, audio_start + audio_count);
      if (a < b) {
        HIPCHK(e, hipMemcpyAsync(e->pf_voice, voice + (size_t)(a - audio_start) * DIM,
                                 (size_t)(b - a) * DIM * 4, hipMemcpyHostToDevice, e->st));
        vs = a;
        vc = b - a;
      }
    }
    if ((rc = enqueue_prefill_chunk(e, n, c0, vs, vc, vc > 0))) return rc;
    LAUNCHCHK(e);
    HIPCHK(e, hipStreamSynchronize(e->st));  // the host buffers above are reused per chunk
  }
  return VX_OK;
}

// sampleTopP, src/engine.ts:247-289 (JS numbers are f64, the arrays f32);
// Math.random replaced by the next draw of a seeded splitmix64 stream
static uint32_t sample_top_p(const float *logits, int n, double top_p, double temp,
                             uint64_t *rng) {
  std::vector<float> sc(n);
  for (int i = 0; i < n; i++) sc[i] = (float)((double)logits[i] / temp);
  double mx = -INFINITY;
  for (int i = 0; i < n; i++)
    if (sc[i] > mx) mx = sc[i];
  double sum = 0;
  for (int i = 0; i < n; i++) {
    sc[i] = (float)std::exp((double)sc[i] - mx);
    sum += sc[i];
  }
  for (int i = 0; i < n; i++) sc[i] = (float)((double)sc[i] / sum);
  std::vector<int> idx(n);
  std::iota(idx.begin(), idx.end(), 0);
  std::stable_sort(idx.begin(), idx.end(), [&](int a, int b) { return sc[b] < sc[a]; });
  double cum = 0;
  int cutoff = n;
  for (int i = 0; i < n; i++) {
    cum += sc[idx[i]];
    if (cum >= top_p) {
      cutoff = i + 1;
      break;
    }
  }
  double resum = 0;
  for (int i = 0; i < cutoff; i++) resum += sc[idx[i]];
  *rng += 0x9E3779B97F4A7C15ull;
  uint64_t z = *rng;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z ^= z >> 31;
  double r = (double)(z >> 11) * 0x1p-53 * resum;
  double acc = 0;
  for (int i = 0; i < cutoff; i++) {
    acc += sc[idx[i]];
    if (acc >= r) return (uint32_t)idx[i];
  }
  return (uint32_t)idx[0];
}

int vx_sample_top_p(vx_engine *e, const float *logits, int32_t n, int32_t valid, double top_p,
                    double temperature, uint64_t *state, int32_t on_device, uint32_t *code) {
  if (!e || !logits || !state || !code) return VX_E_INVALID;
  if (n < 2 || n > TP_MAXN || valid < 2 || !(temperature > 0.0) || !std::isfinite(temperature) ||
      !(top_p > 0.0) || !(top_p <= 1.0))
    return fail(e, VX_E_INVALID, "top-p: n %d, valid %d, temperature %g, top_p %g out of range", n,
                valid, temperature, top_p);
  if (!on_device) {
    std::vector<float> l(logits, logits + n);
    l[0] = -INFINITY;
    for (int i = valid; i < n; i++) l[i] = -INFINITY;
    *code = sample_top_p(l.data(), n, top_p, temperature, state);
    return VX_OK;
  }
  const double params[2] = {top_p, temperature};
  HIPCHK(e, hipMemcpyAsync(e->tp_logits, logits, (size_t)n * 4, hipMemcpyHostToDevice, e->st));
  HIPCHK(e, hipMemcpyAsync(e->tp_params, params, 16, hipMemcpyHostToDevice, e->st));
  HIPCHK(e, hipMemcpyAsync(e->rng_state, state, 8, hipMemcpyHostToDevice, e->st));
  hipLaunchKernelGGL(topp_sample_kernel, dim3(1), dim3(TP_NT), 0, e->st, e->tp_logits, n, valid,
                     e->tp_params, e->rng_state, e->argmax_res, (const int *)nullptr, (uint32_t *)nullptr);
  LAUNCHCHK(e);
  HIPCHK(e, hipMemcpyAsync(code, e->argmax_res, 4, hipMemcpyDeviceToHost, e->st));
  HIPCHK(e, hipMemcpyAsync(state, e->rng_state, 8, hipMemcpyDeviceToHost, e->st));
  HIPCHK(e, hipStreamSynchronize(e->st));
  return VX_OK;
}

// vx_sample_top_p's device path with its staging in the file-scope array
// above: no engine, no allocation.  Runs on the null stream of the current
// device and waits for it.  Calls that overlap on one GPU share the array
// and race.
int vx_sample_top_p_noalloc(const float *logits, int32_t n, int32_t valid, double top_p,
                            double temperature, uint64_t *state, uint32_t *code) {
  if (!logits || !state || !code) return fail(nullptr, VX_E_INVALID, "NULL argument");
  if (n > TP_MAXN)
    return fail(nullptr, VX_E_RANGE,
                "top-p: %d logits exceed the %d of the allocation-free sampler's device buffer", n,
                TP_MAXN);
  if (n < 2 || valid < 2 || !(temperature > 0.0) || !std::isfinite(temperature) ||
      !(top_p > 0.0) || !(top_p <= 1.0))
    return fail(nullptr, VX_E_INVALID, "top-p: n %d, valid %d, temperature %g, top_p %g out of range",
                n, valid, temperature, top_p);
  int dev = 0;
  char *base = noalloc_scratch(&dev);
  if (!base) return VX_E_DEVICE;
  std::lock_guard<std::mutex> call_lock(g_na_call_mu[dev]);
  float *d_logits = (float *)(base + NA_LOGITS);
  double *d_params = (double *)(base + NA_PARAMS);
  uint64_t *d_state = (uint64_t *)(base + NA_STATE);
  uint32_t *d_code = (uint32_t *)(base + NA_CODE);
  const double params[2] = {top_p, temperature};
  hipStream_t st = nullptr;
  // every operand the kernel reads is written first: nothing stale from an
  // earlier call is used
  HIPCHK(nullptr, hipMemcpyAsync(d_logits, logits, (size_t)n * 4, hipMemcpyHostToDevice, st));
  HIPCHK(nullptr, hipMemcpyAsync(d_params, params, sizeof params, hipMemcpyHostToDevice, st));
  HIPCHK(nullptr, hipMemcpyAsync(d_state, state, 8, hipMemcpyHostToDevice, st));
  hipLaunchKernelGGL(topp_sample_kernel, dim3(1), dim3(TP_NT), 0, st, d_logits, n, valid, d_params,
                     d_state, d_code, (const int *)nullptr, (uint32_t *)nullptr);
  LAUNCHCHK(nullptr);
  HIPCHK(nullptr, hipMemcpyAsync(code, d_code, 4, hipMemcpyDeviceToHost, st));
  HIPCHK(nullptr, hipMemcpyAsync(state, d_state, 8, hipMemcpyDeviceToHost, st));
  HIPCHK(nullptr, hipStreamSynchronize(st));
  return VX_OK;
}

// ------------------------------------------------------------- generate
void vx_generate_options_default(vx_generate_options *o) {
  if (!o) return;
  o->sampling = VX_SAMPLE_TOP_P;
  o->top_p = 0.9;
  o->temperature = 0.8;
  o->seed = 0;
  o->ignore_eos = 0;
}

// -------------------------------------------------------- codec decoder
// codecDecode (src/engine.ts:1402-1713) on MFMA GEMMs (vx_codec.h).

// derived operands, rebuilt after any weight change: the normalised VQ
// codebook (normalizeVQCodebook :593-613), the transposed convs' weight-norm
// scales (precomputeConvTransposeScales :621-657), the causal convs' row
// scales, and every conv weight in its GEMM order
static int codec_prepare(vx_engine *e) {
  if (e->codec_ready) return VX_OK;
  const CodecW &w = e->cw;
  hipStream_t st = e->st;
  hipLaunchKernelGGL(cx_vq_norm_kernel, dim3(1024), dim3(256), 0, st, w.cb_sum, w.cb_usage, e->cx_cb);
  hipLaunchKernelGGL(cx_conv_rowscale_kernel, dim3(CD / 64), dim3(64), 0, st, w.in_w, w.in_g, CD,
                     CIN * CK_IN, CD, e->cx_rs_in);
  hipLaunchKernelGGL(cx_conv_rowscale_kernel, dim3(CPATCH_ROWS / 64), dim3(64), 0, st, w.out_w,
                     w.out_g, CPATCH, CKOUT, CPATCH_ROWS, e->cx_rs_out);
  hipLaunchKernelGGL(cx_reorder_in_kernel, dim3(1024), dim3(256), 0, st, w.in_w, e->cx_ain);
  hipLaunchKernelGGL(cx_reorder_out_kernel, dim3(1024), dim3(256), 0, st, w.out_w, e->cx_aout);
  for (int s = 0; s < CX_STAGES - 1; s++) {
    hipLaunchKernelGGL(cx_up_scale_kernel, dim3(CD), dim3(256), 0, st, w.up_w[s], w.up_g[s],
                       e->cx_s_up[s]);
    hipLaunchKernelGGL(cx_reorder_up_kernel, dim3(2048), dim3(256), 0, st, w.up_w[s], e->cx_aup[s]);
  }
  LAUNCHCHK(e);
  HIPCHK(e, hipStreamSynchronize(st));
  e->codec_ready = true;
  return VX_OK;
}

// per-decode buffers for up to T frames (8 T tokens after the upsampling)
static int codec_reserve(vx_engine *e, int T) {
  if (T <= e->cx_cap) return VX_OK;
  if (e->cx_arena) {
    HIPCHK(e, hipStreamSynchronize(e->st));
    HIPCHK(e, hipFree(e->cx_arena));
    e->cx_arena = nullptr;
    e->cx_cap = 0;
  }
  const size_t TT = (size_t)8 * T;
  std::vector<std::pair<void **, size_t>> parts = {
      {(void **)&e->cx_x, TT * CD * 4},
      {(void **)&e->cx_x2, TT * CD * 4},
      {(void **)&e->cx_q, TT * CD * 4},
      {(void **)&e->cx_k, TT * CD * 4},
      {(void **)&e->cx_v, TT * CD * 4},
      {(void **)&e->cx_attn, TT * CD * 4},
      {(void **)&e->cx_audio, TT * CPATCH * 4},
      {(void **)&e->cx_c, CX_CCAP * 4},
      {(void **)&e->cx_b, (size_t)CKOUT / 8 * CX_NC * 16},
      {(void **)&e->cx_sem, (size_t)T * 4},
      {(void **)&e->cx_ac, (size_t)T * NAC * 4}};
  size_t tot = 0;
  for (auto &q : parts) tot += align256(q.second);
  if (hipMalloc(&e->cx_arena, tot) != hipSuccess)
    return fail(e, VX_E_NOMEM, "hipMalloc of %zu codec bytes for %d frames failed", tot, T);
  char *p = (char *)e->cx_arena;
  for (auto &q : parts) {
    *q.first = p;
    p += align256(q.second);
  }
  e->cx_cap = T;
  return VX_OK;
}

// the intermediates of debugCodecDecode (src/engine.ts:1719-1985)
static int cx_stop_frames(int T, int stop) {
  if (stop <= VX_CODEC_STOP_STAGE0) return T;
  if (stop == VX_CODEC_STOP_AUDIO) return 8 * T;
  const int s = (stop - VX_CODEC_STOP_STAGE0) / 2, up = (stop - VX_CODEC_STOP_STAGE0) % 2;
  return T << (s + up);
}

// codes already in cx_sem / cx_ac; enqueues the decoder up to `stop` and
// leaves the result in *res (device) with *count floats
static int codec_run(vx_engine *e, int T, int stop, const float **res, size_t *count) {
  hipStream_t st = e->st;
  int rc = VX_OK;  // the first GEMM failure; later launches only queue work
  const CodecW &w = e->cw;
  const int levels = e->cfg.acoustic_levels;
  const dim3 blk(256);
  // token chunks [t0, t0 + n) with nc = 2 * round_up(n, 128) B columns
  auto chunks = [&](int TT, auto &&body) {
    for (int t0 = 0; t0 < TT; t0 += e->cx_chunk) {
      const int n = std::min(e->cx_chunk, TT - t0), nc = 2 * ((n + 127) / 128 * 128);
      body(t0, n, nc);
    }
  };
  if (stop == VX_CODEC_STOP_CONCAT) {
    hipLaunchKernelGGL(cx_concat_kernel, dim3((T * CIN + 255) / 256), blk, 0, st, e->cx_cb,
                       e->cx_sem, e->cx_ac, levels, T, e->cx_x);
    *res = e->cx_x;
    *count = (size_t)T * CIN;
    return VX_OK;
  }
  // input conv: CausalConv1d(292 -> 1024, k = 3)
  chunks(T, [&](int t0, int n, int nc) {
    hipLaunchKernelGGL(cx_pack_in_kernel, dim3(nc / 2), dim3(128), 0, st, e->cx_cb, e->cx_sem,
                       e->cx_ac, levels, t0, n, nc, e->cx_b);
    int ns = 1;
    if (!rc) rc = cx_gemm(e, e->cx_ain, CD, CKIN, nc, &ns);
    gm_with_slices(ns, [&](auto NS) {
      hipLaunchKernelGGL(cx_scale_rows_epi_kernel<NS>, dim3(n, CD / 256), blk, 0, st, e->cx_c, CD, nc, t0,
                         e->cx_rs_in, CD, e->cx_x, CD);
    });
  });
  int TT = T, at = VX_CODEC_STOP_INPUT_CONV;
  float *x = e->cx_x, *x2 = e->cx_x2;
  static const int kWindow[CX_STAGES] = {2, 4, 8, 16};  // src/engine.ts:1507
  for (int s = 0; s < CX_STAGES && at < stop; s++) {
    for (int l = 0; l < CX_LPS; l++) {
      const CodecLayerW &L = w.L[s][l];
      chunks(TT, [&](int t0, int n, int nc) {
        hipLaunchKernelGGL(cx_pack_kernel<true>, dim3(nc / 2), blk, 0, st, x, CD, t0, n, nc,
                           L.attn_norm, CX_NORM_EPS, e->cx_b);
        int ns = 1;
        if (!rc) rc = cx_gemm(e, L.wqkv, 3 * CD, CD, nc, &ns);
        gm_with_slices(ns, [&](auto NS) {
          hipLaunchKernelGGL(cx_qkv_epi_kernel<NS>, dim3(n, 3 * CNH / 4), blk, 0, st, e->cx_c, nc, t0,
                             L.q_norm, L.k_norm, e->cx_q, e->cx_k, e->cx_v);
        });
      });
      hipLaunchKernelGGL(cx_attn_kernel, dim3(TT, CNH / 4), blk, 0, st, e->cx_q, e->cx_k, e->cx_v,
                         kWindow[s], e->cx_attn);
      chunks(TT, [&](int t0, int n, int nc) {
        hipLaunchKernelGGL(cx_pack_kernel<false>, dim3(nc / 2), blk, 0, st, e->cx_attn, CD, t0, n,
                           nc, nullptr, 0.f, e->cx_b);
        int ns = 1;
        if (!rc) rc = cx_gemm(e, L.wo, CD, CD, nc, &ns);
        gm_with_slices(ns, [&](auto NS) {
          hipLaunchKernelGGL(cx_resid_epi_kernel<NS>, dim3(n, CD / 256), blk, 0, st, e->cx_c, nc, t0,
                             L.attn_scale, x);
        });
      });
      chunks(TT, [&](int t0, int n, int nc) {
        hipLaunchKernelGGL(cx_pack_kernel<true>, dim3(nc / 2), blk, 0, st, x, CD, t0, n, nc,
                           L.ffn_norm, CX_NORM_EPS, e->cx_b);
        int ns = 1;
        if (!rc) rc = cx_gemm(e, L.w13, 2 * CHID, CD, nc, &ns);
        // the gate/up GEMM has consumed B: the SwiGLU epilogue refills it
        gm_with_slices(ns, [&](auto NS) {
          hipLaunchKernelGGL(cx_swiglu_epi_kernel<NS>, dim3(nc / 2, CHID / 8 / 256), blk, 0, st, e->cx_c,
                             nc, n, e->cx_b);
        });
        if (!rc) rc = cx_gemm(e, L.w2, CD, CHID, nc, &ns);
        gm_with_slices(ns, [&](auto NS) {
          hipLaunchKernelGGL(cx_resid_epi_kernel<NS>, dim3(n, CD / 256), blk, 0, st, e->cx_c, nc, t0,
                             L.ffn_scale, x);
        });
      });
    }
    at = VX_CODEC_STOP_STAGE0 + 2 * s;
    if (at == stop || s == CX_STAGES - 1) break;
    // ConvTranspose1d(1024 -> 1024, k = 4, stride 2), output trimmed to 2 TT
    chunks(TT, [&](int t0, int n, int nc) {
      hipLaunchKernelGGL(cx_pack_up_kernel, dim3(nc / 2), blk, 0, st, x, e->cx_s_up[s], t0, n, nc,
                         e->cx_b);
      int ns = 1;
      if (!rc) rc = cx_gemm(e, e->cx_aup[s], 2 * CD, CKUP, nc, &ns);
      gm_with_slices(ns, [&](auto NS) {
        hipLaunchKernelGGL(cx_up_epi_kernel<NS>, dim3(n, 2 * CD / 256), blk, 0, st, e->cx_c, nc, t0, x2);
      });
    });
    std::swap(x, x2);
    TT *= 2;
    at = VX_CODEC_STOP_STAGE0 + 2 * s + 1;
  }
  if (rc) return rc;
  if (stop != VX_CODEC_STOP_AUDIO) {
    *res = x;
    *count = (size_t)TT * CD;
    return VX_OK;
  }
  // output conv: CausalConv1d(1024 -> 240, k = 7); step t gives samples
  // [240 t, 240 t + 240)
  chunks(TT, [&](int t0, int n, int nc) {
    hipLaunchKernelGGL(cx_pack_out_kernel, dim3(nc / 2), blk, 0, st, x, t0, n, nc, e->cx_b);
    int ns = 1;
    if (!rc) rc = cx_gemm(e, e->cx_aout, CPATCH_ROWS, CKOUT, nc, &ns);
    gm_with_slices(ns, [&](auto NS) {
      hipLaunchKernelGGL(cx_scale_rows_epi_kernel<NS>, dim3(n, 1), blk, 0, st, e->cx_c, CPATCH_ROWS, nc,
                         t0, e->cx_rs_out, CPATCH, e->cx_audio, CPATCH);
    });
  });
  if (rc) return rc;
  *res = e->cx_audio;
  *count = (size_t)TT * CPATCH;
  return VX_OK;
}

static int codec_decode_impl(vx_engine *e, const uint32_t *semantic, const uint32_t *acoustic,
                             int32_t n_frames, int32_t stop, float *out, size_t out_count) {
  if (!e) return VX_E_INVALID;
  if (!e->codec_on) return fail(e, VX_E_STATE, "the engine was created without the codec decoder");
  int rc = check_ready(e);
  if (rc) return fail(e, VX_E_STATE, "Engine not initialized. Call init() and loadWeights() first.");
  if (n_frames < 1 || n_frames > VX_CODEC_MAX_FRAMES || !semantic || !acoustic || !out ||
      stop < VX_CODEC_STOP_CONCAT || stop > VX_CODEC_STOP_AUDIO)
    return fail(e, VX_E_INVALID, "bad codec arguments (frames %d, stop %d)", n_frames, stop);
  if (out_count < vx_codec_stop_count(n_frames, stop))
    return fail(e, VX_E_INVALID, "output holds %zu floats, %zu needed", out_count,
                vx_codec_stop_count(n_frames, stop));
  if ((rc = codec_prepare(e)) || (rc = codec_reserve(e, n_frames)) || (rc = pf_gemm_setup(e)))
    return rc;
  HIPCHK(e, hipMemcpyAsync(e->cx_sem, semantic, (size_t)n_frames * 4, hipMemcpyHostToDevice, e->st));
  HIPCHK(e, hipMemcpyAsync(e->cx_ac, acoustic, (size_t)n_frames * NAC * 4, hipMemcpyHostToDevice,
                           e->st));
  const float *res = nullptr;
  size_t count = 0;
  if ((rc = codec_run(e, n_frames, stop, &res, &count))) return rc;
  LAUNCHCHK(e);
  HIPCHK(e, hipMemcpyAsync(out, res, count * 4, hipMemcpyDeviceToHost, e->st));
  HIPCHK(e, hipStreamSynchronize(e->st));
  return VX_OK;
}

size_t vx_codec_stop_count(int32_t n_frames, int32_t stop) {
  if (n_frames < 0 || stop < VX_CODEC_STOP_CONCAT || stop > VX_CODEC_STOP_AUDIO) return 0;
  const size_t f = (size_t)cx_stop_frames(n_frames, stop);
  return f * (stop == VX_CODEC_STOP_CONCAT ? CIN : stop == VX_CODEC_STOP_AUDIO ? CPATCH : CD);
}

int vx_codec_decode(vx_engine *e, const uint32_t *semantic, const uint32_t *acoustic,
                    int32_t n_frames, float *audio) {
  return codec_decode_impl(e, semantic, acoustic, n_frames, VX_CODEC_STOP_AUDIO, audio,
                           vx_codec_stop_count(n_frames, VX_CODEC_STOP_AUDIO));
}

int vx_codec_decode_debug(vx_engine *e, const uint32_t *semantic, const uint32_t *acoustic,
                          int32_t n_frames, int32_t stop, float *out, size_t out_count) {
  return codec_decode_impl(e, semantic, acoustic, n_frames, stop, out, out_count);
}

// sampleTopP, src/engine.ts:247-289, with a seeded uniform in place of
// Math.random.  Float32Array intermediates, double accumulators, stable
// descending sort, as the TypeScript does.
// splitmix64 increment: the device top-p stream advances by it once per frame
constexpr uint64_t kTopPGamma = 0x9E3779B97F4A7C15ull;

// Puts back the state frame f left when generate() discards the speculative
// frame f + 1 after frame f's EOS: the position (frame f + 1's step), the
// residual stream, normed and the semantic logits (saved by frame f + 1's
// first kernel), frame f's codes, the FM frame counter (f + 1 frames drew
// noise) and the top-p generator state rng.  Frame f + 1's K/V row lies past
// the position and is never read.
static int undo_frame(vx_engine *e, int f, uint32_t code, const uint32_t *codes, uint64_t rng) {
  int rc = vx_set_position(e, e->host_pos - 1);
  if (rc) return rc;
  HIPCHK(e, hipMemcpyAsync(e->x, e->x_prev, DIM * 4, hipMemcpyDeviceToDevice, e->st));
  HIPCHK(e, hipMemcpyAsync(e->normed, e->normed_prev, DIM * 4, hipMemcpyDeviceToDevice, e->st));
  HIPCHK(e, hipMemcpyAsync(e->sem_logits, e->logits_prev, SEMV * 4, hipMemcpyDeviceToDevice, e->st));
  HIPCHK(e, hipMemcpyAsync(e->sem_code, &code, 4, hipMemcpyHostToDevice, e->st));
  HIPCHK(e, hipMemcpyAsync(e->codes, codes, NAC * 4, hipMemcpyHostToDevice, e->st));
  HIPCHK(e, hipMemcpyAsync(e->rng_state, &rng, 8, hipMemcpyHostToDevice, e->st));
  hipLaunchKernelGGL(set_int_kernel, dim3(1), dim3(1), 0, e->st, e->frame, f + 1);
  LAUNCHCHK(e);
  HIPCHK(e, hipStreamSynchronize(e->st));
  return VX_OK;
}

int vx_generate(vx_engine *e, const int32_t *tokens, int32_t n_tokens, int32_t audio_start,
                int32_t audio_count, const float *voice, int32_t max_frames,
                const vx_generate_options *opt_in, vx_frame_cb on_frame, vx_stage_cb on_stage,
                void *user, uint32_t *sem_out, uint32_t *ac_out, float *audio_out,
                vx_generate_stats *stats) {
  if (!e) return VX_E_INVALID;
  if (audio_out && !e->codec_on)
    return fail(e, VX_E_STATE, "the engine was created without the codec decoder");
  int rc = check_ready(e);
  if (rc) return fail(e, VX_E_STATE, "Engine not initialized. Call init() and loadWeights() first.");
  if (n_tokens < 0 || (n_tokens > 0 && !tokens) || max_frames < 0)
    return fail(e, VX_E_INVALID, "bad arguments");
  if ((int64_t)n_tokens + 1 + (max_frames > 0 ? max_frames - 1 : 0) > e->max_seq)
    return fail(e, VX_E_RANGE, "prompt + frames exceed max_seq_len %d", e->max_seq);
  vx_generate_options opt;
  vx_generate_options_default(&opt);
  if (opt_in) opt = *opt_in;
  if (opt.sampling != VX_SAMPLE_GREEDY && opt.sampling != VX_SAMPLE_TOP_P &&
      opt.sampling != VX_SAMPLE_TOP_P_HOST)
    return fail(e, VX_E_INVALID, "unknown sampling mode %d", opt.sampling);
  // NaN fails both comparisons
  if (opt.sampling != VX_SAMPLE_GREEDY &&
      (!(opt.temperature > 0.0) || !std::isfinite(opt.temperature) || !(opt.top_p > 0.0) ||
       !(opt.top_p <= 1.0)))
    return fail(e, VX_E_INVALID, "top-p sampling needs temperature > 0 and top_p in (0, 1] "
                "(temperature %g, top_p %g)", opt.temperature, opt.top_p);
  if (audio_count < 0 || (audio_count > 0 && audio_start < 0) ||
      (int64_t)audio_start + audio_count > INT32_MAX)
    return fail(e, VX_E_INVALID, "bad voice range (start %d, count %d)", audio_start, audio_count);
  using clk = std::chrono::steady_clock;
  auto ms = [](clk::time_point a, clk::time_point b) {
    return std::chrono::duration<double, std::milli>(b - a).count();
  };
  if ((rc = vx_reset(e))) return rc;
  std::vector<uint32_t> sem_v, ac_v;  // the codes, for the codec decode
  if (audio_out) {
    sem_v.reserve(max_frames);
    ac_v.reserve((size_t)max_frames * NAC);
  }
  HIPCHK(e, hipMemcpyAsync(e->noise_seed, &opt.seed, 8, hipMemcpyHostToDevice, e->st));
  HIPCHK(e, hipStreamSynchronize(e->st));
  auto t0 = clk::now();
  if (on_stage) on_stage(user, 0, -1.0);
  if ((rc = ensure_tproj(e))) return rc;
  // prefill (src/engine.ts:2457-2472) as batched GEMMs, chunk by chunk; the
  // LM head the reference runs per prefill token is never read, so it is
  // skipped
  if (n_tokens > 0 && (rc = vx_prefill(e, tokens, n_tokens, audio_start, audio_count, voice)))
    return rc;
  HIPCHK(e, hipStreamSynchronize(e->st));
  auto t1 = clk::now();
  if (on_stage) {
    on_stage(user, 0, ms(t0, t1));
    on_stage(user, 1, -1.0);
  }
  // AUDIO token kick (src/engine.ts:2478-2487)
  if ((rc = prepare_input(e, 24, VX_EMBED_TOKEN, nullptr))) return rc;
  if ((rc = run_step(e))) return rc;
  e->host_pos++;

  uint64_t rng = opt.seed ^ 0x5bd1e9955bd1e995ull;
  const double params[2] = {opt.top_p, opt.temperature};
  HIPCHK(e, hipMemcpyAsync(e->rng_state, &rng, 8, hipMemcpyHostToDevice, e->st));
  HIPCHK(e, hipMemcpyAsync(e->tp_params, params, 16, hipMemcpyHostToDevice, e->st));
  int frames = 0;
  if (opt.sampling == VX_SAMPLE_TOP_P_HOST) {
    // the reference's dataflow: logits to the host every frame
    std::vector<float> logits(SEMV);
    uint32_t codes[NAC];
    for (int f = 0; f < max_frames; f++) {
      if (f > 0) {
        if ((rc = prepare_input(e, 0, VX_EMBED_CODES, nullptr))) return rc;
        if ((rc = run_step(e))) return rc;
        e->host_pos++;
      }
      if ((rc = run_seq(e, &e->fm_plain_exec, fm_plain_body))) return rc;
      HIPCHK(e, hipMemcpyAsync(logits.data(), e->sem_logits, SEMV * 4, hipMemcpyDeviceToHost, e->st));
      HIPCHK(e, hipStreamSynchronize(e->st));
      logits[0] = -INFINITY;  // src/engine.ts:2559-2563
      for (int i = 8194; i < SEMV; i++) logits[i] = -INFINITY;
      const uint32_t code = sample_top_p(logits.data(), SEMV, opt.top_p, opt.temperature, &rng);
      if (code <= 1 && !opt.ignore_eos) break;
      hipLaunchKernelGGL(set_u32_kernel, dim3(1), dim3(1), 0, e->st, e->sem_code, code);
      LAUNCHCHK(e);
      HIPCHK(e, hipMemcpyAsync(codes, e->codes, NAC * 4, hipMemcpyDeviceToHost, e->st));
      HIPCHK(e, hipStreamSynchronize(e->st));
      if (sem_out) sem_out[f] = code;
      if (ac_out) memcpy(ac_out + (size_t)f * NAC, codes, sizeof codes);
      if (audio_out) {
        sem_v.push_back(code);
        ac_v.insert(ac_v.end(), codes, codes + NAC);
      }
      frames++;
      if (on_frame) on_frame(user, f, code, codes);
    }
  } else {
    // codes stay on the device: frame f + 1 (multi-codebook embed of frame
    // f's codes, backbone step, FM, sampling) is enqueued before frame f's
    // codes are read back through pinned memory, so the host work of frame
    // f (EOS test, callback) overlaps frame f + 1 on the GPU.  If frame f
    // ends the utterance, frame f + 1 is discarded: its KV row lies past the
    // position the engine is left at and is never read.
    const bool greedy = opt.sampling == VX_SAMPLE_GREEDY;
    hipGraphExec_t *fm_slot = greedy ? &e->fm_greedy_exec : &e->fm_topp_exec;
    hipGraphExec_t *frame_slot = greedy ? &e->frame_exec : &e->frame_topp_exec;
    void (*fm_body)(vx_engine *) = greedy ? fm_greedy_body : fm_topp_body;
    void (*fr_body)(vx_engine *) = greedy ? frame_body : frame_topp_body;
    // frame f's last kernels store its codes into host slot f & 1 (the
    // device frame counter is f there: vx_reset zeroed it and each frame's
    // fm_finish_kernel advances it), so the host only waits for its event
    auto enqueue_frame = [&](int f) -> int {
      int r = f == 0 ? run_seq(e, fm_slot, fm_body) : run_seq(e, frame_slot, fr_body);
      if (r) return r;
      HIPCHK(e, hipEventRecord(e->ev_frame[f & 1], e->st));
      return VX_OK;
    };
    if (max_frames > 0 && (rc = enqueue_frame(0))) return rc;
    for (int f = 0; f < max_frames; f++) {
      const bool ahead = f + 1 < max_frames;
      if (ahead) {
        if ((rc = enqueue_frame(f + 1))) return rc;
        e->host_pos++;  // the backbone step of frame f + 1
      }
      HIPCHK(e, hipEventSynchronize(e->ev_frame[f & 1]));
      const uint32_t *slot = e->h_frame + (f & 1) * (1 + NAC);
      const uint32_t code = slot[0];
      uint32_t codes[NAC];
      memcpy(codes, slot + 1, sizeof codes);
      if (code <= 1 && !opt.ignore_eos) {
        if (ahead) {  // undo the speculative frame f + 1
          HIPCHK(e, hipStreamSynchronize(e->st));
          if ((rc = undo_frame(e, f, code, codes, greedy ? rng : rng + (uint64_t)(f + 1) * kTopPGamma)))
            return rc;
        }
        break;
      }
      if (sem_out) sem_out[f] = code;
      if (ac_out) memcpy(ac_out + (size_t)f * NAC, codes, sizeof codes);
      if (audio_out) {
        sem_v.push_back(code);
        ac_v.insert(ac_v.end(), codes, codes + NAC);
      }
      frames++;
      if (on_frame) on_frame(user, f, code, codes);
    }
  }
  HIPCHK(e, hipStreamSynchronize(e->st));
  auto t2 = clk::now();
  if (on_stage) {
    on_stage(user, 1, ms(t1, t2));
    on_stage(user, 2, -1.0);
  }
  // codec decode of all frames (src/engine.ts:2588-2599)
  if (audio_out && frames > 0 &&
      (rc = vx_codec_decode(e, sem_v.data(), ac_v.data(), frames, audio_out)))
    return rc;
  auto t3 = clk::now();
  if (on_stage) on_stage(user, 2, ms(t2, t3));
  if (stats) {
    stats->backbone_ms = ms(t0, t1);
    stats->fm_ms = ms(t1, t2);
    stats->codec_ms = ms(t2, t3);
    stats->total_ms = ms(t0, t3);
    stats->frames_generated = frames;
  }
  HIPCHK(e, hipStreamSynchronize(e->st));
  return VX_OK;
}

// ------------------------------------------------------------ tokenizer
int vx_tokenizer_create(const uint8_t *blob, const int64_t *offsets, const int32_t *ranks,
                        int32_t n, int32_t num_special, vx_tokenizer **out) {
  if (!out) return fail(nullptr, VX_E_INVALID, "out is NULL");
  *out = nullptr;
  if (n < 0 || (n > 0 && (!blob || !offsets || !ranks)) || num_special < 0)
    return fail(nullptr, VX_E_INVALID, "bad tokenizer vocabulary arguments");
  auto *t = new vx_tokenizer{BpeVocab(num_special)};
  for (int32_t i = 0; i < n; i++) {
    if (offsets[i] < 0 || offsets[i + 1] < offsets[i] || ranks[i] < 0) {
      delete t;
      return fail(nullptr, VX_E_INVALID, "vocabulary entry %d is malformed", i);
    }
    t->vocab.add(blob + offsets[i], (size_t)(offsets[i + 1] - offsets[i]), ranks[i]);
  }
  *out = t;
  return VX_OK;
}

void vx_tokenizer_destroy(vx_tokenizer *t) { delete t; }

int vx_tokenizer_encode_pieces(const vx_tokenizer *t, const uint8_t *bytes,
                               const int64_t *offsets, int32_t n_pieces, int32_t *out, int64_t cap,
                               int64_t *n_out) {
  if (!t || n_pieces < 0 || (n_pieces > 0 && (!bytes || !offsets)) || !n_out || cap < 0 ||
      (cap > 0 && !out))
    return fail(nullptr, VX_E_INVALID, "bad tokenizer arguments");
  std::vector<int32_t> ids;
  for (int32_t j = 0; j < n_pieces; j++) {
    if (offsets[j] < 0 || offsets[j + 1] < offsets[j])
      return fail(nullptr, VX_E_INVALID, "piece %d is malformed", j);
    t->vocab.encode(bytes + offsets[j], (size_t)(offsets[j + 1] - offsets[j]), ids);
  }
  *n_out = (int64_t)ids.size();
  if ((int64_t)ids.size() > cap)
    return fail(nullptr, VX_E_RANGE, "%zu token ids, room for %lld", ids.size(), (long long)cap);
  std::copy(ids.begin(), ids.end(), out);
  return VX_OK;
}

// ---------------------------------------------------------- measurement
int vx_time_backbone_steps(vx_engine *e, int32_t n, int32_t mode, float *out_ms) {
  if (!e || n < 1 || !out_ms || mode < VX_TIME_ADVANCE || mode > VX_TIME_FEEDBACK)
    return e ? fail(e, VX_E_INVALID, "bad timing arguments") : VX_E_INVALID;
  int rc = check_ready(e);
  if (rc) return rc;
  const bool hold = mode == VX_TIME_HOLD;
  if ((int64_t)e->host_pos + (hold ? 1 : n) > e->max_seq)
    return fail(e, VX_E_RANGE, "steps pass max_seq_len");
  HIPCHK(e, hipEventRecord(e->ev0, e->st));
  for (int i = 0; i < n; i++) {
    rc = hold ? run_step_hold(e)
              : mode == VX_TIME_FEEDBACK ? run_seq(e, &e->feedback_exec, enqueue_backbone_feedback)
                                         : run_step(e);
    if (rc) return rc;
  }
  HIPCHK(e, hipEventRecord(e->ev1, e->st));
  HIPCHK(e, hipEventSynchronize(e->ev1));
  if (!hold) e->host_pos += n;
  HIPCHK(e, hipEventElapsedTime(out_ms, e->ev0, e->ev1));
  return VX_OK;
}

// every slot to (start ~0, end 0): slots of blocks a launch does not have
// drop out of the host's min / max
__global__ void timeline_reset_kernel(unsigned long long *ts, size_t slots) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < slots; i += (size_t)gridDim.x * blockDim.x) {
    ts[2 * i] = ~0ull;
    ts[2 * i + 1] = 0ull;
  }
}

int vx_debug_timeline(vx_engine *e, int32_t reps, uint64_t *stamps, int32_t cap, int32_t *n_out) {
  if (!e || reps < 1 || !stamps || !n_out) return e ? fail(e, VX_E_INVALID, "bad timeline arguments") : VX_E_INVALID;
  int rc = check_ready(e);
  if (rc) return rc;
  const int n = 6 * e->cfg.n_layers + 1;
  *n_out = n;
  if (cap < 2 * n) return fail(e, VX_E_RANGE, "timeline: %d stamps, room for %d", 2 * n, cap);
  if (e->host_pos >= e->max_seq)
    return fail(e, VX_E_RANGE, "position %d reaches max_seq_len %d", e->host_pos, e->max_seq);
  const size_t slots = (size_t)n * TS_BLOCKS;
  for (int r = 0; r < reps; r++) {
    hipLaunchKernelGGL(timeline_reset_kernel, dim3(256), dim3(256), 0, e->st, e->timeline, slots);
    LAUNCHCHK(e);
    if ((rc = run_seq(e, &e->timeline_exec, enqueue_backbone_timeline))) return rc;
  }
  std::vector<uint64_t> all(2 * slots);
  HIPCHK(e, hipMemcpyAsync(all.data(), e->timeline, slots * 16, hipMemcpyDeviceToHost, e->st));
  HIPCHK(e, hipStreamSynchronize(e->st));
  for (int i = 0; i < n; i++) {
    uint64_t s0 = ~0ull, s1 = 0;
    for (int b = 0; b < TS_BLOCKS; b++) {
      s0 = std::min(s0, all[((size_t)i * TS_BLOCKS + b) * 2]);
      s1 = std::max(s1, all[((size_t)i * TS_BLOCKS + b) * 2 + 1]);
    }
    stamps[2 * i] = s0;
    stamps[2 * i + 1] = s1;
  }
  return VX_OK;
}

int vx_time_frames(vx_engine *e, int32_t n, float *out_ms) {
  if (!e || n < 1 || !out_ms) return VX_E_INVALID;
  int rc = check_ready(e);
  if (rc) return rc;
  if ((int64_t)e->host_pos + n > e->max_seq) return fail(e, VX_E_RANGE, "frames pass max_seq_len");
  if ((rc = ensure_tproj(e))) return rc;
  if (e->use_graphs && !e->frame_exec && (rc = capture(e, &e->frame_exec, frame_body)))
    return rc;
  HIPCHK(e, hipEventRecord(e->ev0, e->st));
  for (int i = 0; i < n; i++) {
    if ((rc = run_seq(e, &e->frame_exec, frame_body))) return rc;
  }
  HIPCHK(e, hipEventRecord(e->ev1, e->st));
  HIPCHK(e, hipEventSynchronize(e->ev1));
  e->host_pos += n;
  HIPCHK(e, hipEventElapsedTime(out_ms, e->ev0, e->ev1));
  return VX_OK;
}

int vx_time_kernel(vx_engine *e, int32_t kernel, int32_t iters, float *avg_us, double *bytes) {
  if (!e || iters < 1 || !avg_us || kernel < 0 || kernel > VX_KERNEL_FM_STEP_IN) return VX_E_INVALID;
  int rc = check_ready(e);
  if (rc) return rc;
  if (kernel >= VX_KERNEL_FM_QKV) {
    // one full FM pass first, so every FM buffer holds the values a frame has
    if ((rc = ensure_tproj(e))) return rc;
    enqueue_fm(e, e->noise, true);
    const double fm_b[] = {
        (double)QKV_ROWS * DIM * 2 + DIM * BCOL * 2 + 6.0 * QKV_ROWS * 4,
        6.0 * (QD + 2 * KVD) * 4 + 6.0 * QD * 4 + QD * BCOL * 2,
        (double)DIM * QD * 2 + QD * BCOL * 2 + 6.0 * DIM * 8 + DIM * BCOL * 2,
        2.0 * HID * DIM * 2 + DIM * BCOL * 2 + 6.0 * HID * 4 + HID * BCOL * 2,
        (double)DIM * HID * 2 + HID * BCOL * 2 + 6.0 * DIM * 8 + DIM * BCOL * 2,
        (double)DIM * NAC * 2 + 2.0 * NAC * SSQ_MAX * 4 + 6.0 * DIM * 4 + DIM * BCOL * 2 + 2.0 * DIM * 4,
    };
    const int k = kernel - VX_KERNEL_FM_QKV;
    if (bytes) *bytes = fm_b[k];
    auto launch = [&](int i) {
      const int l = i % e->cfg.fm_layers;
      const int ns = e->nsteps();  // steps >= 1 read the previous step's partials
      if (k == 5) enqueue_fm_step_in(e, ns > 1 ? 1 + i % (ns - 1) : 0, e->noise);
      else enqueue_fm_kernel(e, l, k, l == 0 ? DIM / 256 : DIM / FTR);
    };
    for (int i = 0; i < 2; i++) launch(i);  // warm-up
    HIPCHK(e, hipEventRecord(e->ev0, e->st));
    for (int i = 0; i < iters; i++) launch(i);
    HIPCHK(e, hipEventRecord(e->ev1, e->st));
    LAUNCHCHK(e);
    HIPCHK(e, hipEventSynchronize(e->ev1));
    float ms;
    HIPCHK(e, hipEventElapsedTime(&ms, e->ev0, e->ev1));
    *avg_us = ms * 1000.0f / iters;
    return VX_OK;
  }
  if (e->host_pos >= e->max_seq)
    return fail(e, VX_E_RANGE, "position %d reaches max_seq_len %d", e->host_pos, e->max_seq);
  const double seq = (double)e->host_pos + 1.0;
  const double b[] = {
      (double)QKV_ROWS * DIM * 2 + DIM * 2 + DIM * 4 + QD * 4 + 2.0 * KVD * e->kv_elem,
      seq * KVD * 2 * (double)e->kv_elem + QD * 4 * 2,
      (double)DIM * QD * 2 + QD * 4 + DIM * 8,
      2.0 * HID * DIM * 2 + DIM * 2 + DIM * 4 + HID * 4,
      (double)DIM * HID * 2 + HID * 4 + DIM * 8,
  };
  if (bytes) *bytes = b[kernel];
  for (int i = 0; i < 2; i++) enqueue_layer(e, i % e->cfg.n_layers, kernel);  // warm-up
  HIPCHK(e, hipEventRecord(e->ev0, e->st));
  for (int i = 0; i < iters; i++) enqueue_layer(e, i % e->cfg.n_layers, kernel);
  HIPCHK(e, hipEventRecord(e->ev1, e->st));
  LAUNCHCHK(e);
  HIPCHK(e, hipEventSynchronize(e->ev1));
  float ms;
  HIPCHK(e, hipEventElapsedTime(&ms, e->ev0, e->ev1));
  *avg_us = ms * 1000.0f / iters;
  return VX_OK;
}

}  // extern "C"
