// vx_blas.h -- plain f16 x f16 -> f32 GEMMs through hipBLASLt (host code).
// The batched prefill and the codec decoder multiply f16 weights by their
// activations in the hi/lo f16 form: C = W x B with W [M][K] row-major and
// B holding N columns of K halves each (column n at B + n K).  The result
// C is [N][M] (column n at C + n M), f32.  Nothing is fused into these
// products, so they go to the library; the per-token epilogues stay
// hand-written.
//
// One plan per (M, K, N), made on first use.  By default it is the
// heuristic's first candidate: that choice depends only on the library and
// the device, so every process computes bit-identical products (different
// algorithms sum K in different orders).  With `tune`, the heuristic's
// candidates are each timed on the caller's stream and the fastest is kept,
// which may differ from process to process.
#pragma once
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt-ext.hpp>
#include <hipblaslt/hipblaslt.h>

#include <cstdio>
#include <cstdlib>
#include <map>
#include <string>
#include <tuple>

namespace vx {

class BlasGemm {
 public:
  ~BlasGemm() { release(); }

  // "" on success, else the failing call
  std::string init(size_t workspace_bytes, bool tune) {
    if (h_) return "";
    tune_ = tune;
    const char *lg = getenv("VX_BLAS_LOG");  // print each new plan's algorithm on stderr
    log_ = lg && atoi(lg) != 0;
    if (hipblasLtCreate(&h_) != HIPBLAS_STATUS_SUCCESS) {
      h_ = nullptr;
      return "hipblasLtCreate failed";
    }
    if (hipMalloc(&ws_, workspace_bytes) != hipSuccess) {
      ws_ = nullptr;
      return "hipMalloc of the GEMM workspace failed";
    }
    wsz_ = workspace_bytes;
    return "";
  }

  void release() {
    for (auto &p : plans_) destroy(p.second);
    plans_.clear();
    if (ws_) (void)hipFree(ws_);
    ws_ = nullptr;
    if (h_) hipblasLtDestroy(h_);
    h_ = nullptr;
  }

  // C[n][m] = sum_k W[m][k] B[n][k]; "" on success
  std::string gemm(const uint16_t *W, int M, int K, const uint16_t *B, int N, float *C,
                   hipStream_t st) {
    if (!h_) return "the GEMM library is not initialised";
    Plan *p = nullptr;
    std::string err = plan(M, K, N, W, B, C, st, &p);
    if (!err.empty()) return err;
    const float alpha = 1.f, beta = 0.f;
    if (hipblasLtMatmul(h_, p->d, &alpha, W, p->la, B, p->lb, &beta, C, p->lc, C, p->lc, &p->algo,
                        ws_, wsz_, st) != HIPBLAS_STATUS_SUCCESS)
      return "hipblasLtMatmul failed";
    return "";
  }

 private:
  struct Plan {
    hipblasLtMatmulDesc_t d;
    hipblasLtMatrixLayout_t la, lb, lc;
    hipblasLtMatmulAlgo_t algo;
  };
  static void destroy(Plan &p) {
    if (p.la) hipblasLtMatrixLayoutDestroy(p.la);
    if (p.lb) hipblasLtMatrixLayoutDestroy(p.lb);
    if (p.lc) hipblasLtMatrixLayoutDestroy(p.lc);
    if (p.d) hipblasLtMatmulDescDestroy(p.d);
  }
  hipblasLtHandle_t h_ = nullptr;
  bool tune_ = false, log_ = false;
  void *ws_ = nullptr;
  size_t wsz_ = 0;
  std::map<std::tuple<int, int, int>, Plan> plans_;

  std::string plan(int M, int K, int N, const uint16_t *W, const uint16_t *B, float *C,
                   hipStream_t st, Plan **out) {
    auto key = std::make_tuple(M, K, N);
    auto it = plans_.find(key);
    if (it != plans_.end()) {
      *out = &it->second;
      return "";
    }
    Plan p{};
    // column-major view: W is K x M (ld K) used transposed; B is K x N
    // (ld K); C is M x N (ld M)
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    if (hipblasLtMatmulDescCreate(&p.d, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatmulDescSetAttribute(p.d, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof ta) !=
            HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatmulDescSetAttribute(p.d, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof tb) !=
            HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&p.la, HIP_R_16F, K, M, K) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&p.lb, HIP_R_16F, K, N, K) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&p.lc, HIP_R_32F, M, N, M) != HIPBLAS_STATUS_SUCCESS) {
      destroy(p);
      return "hipBLASLt descriptor creation failed";
    }
    hipblasLtMatmulPreference_t pref;
    if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) {
      destroy(p);
      return "hipBLASLt preference creation failed";
    }
    hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsz_,
                                          sizeof wsz_);
    constexpr int NC = 8;
    hipblasLtMatmulHeuristicResult_t res[NC];
    int got = 0;
    const hipblasStatus_t hs = hipblasLtMatmulAlgoGetHeuristic(h_, p.d, p.la, p.lb, p.lc, p.lc,
                                                               pref, tune_ ? NC : 1, res, &got);
    hipblasLtMatmulPreferenceDestroy(pref);
    if (hs != HIPBLAS_STATUS_SUCCESS || got < 1) {
      destroy(p);
      return "no hipBLASLt algorithm for this GEMM";
    }
    if (!tune_) {
      p.algo = res[0].algo;
      note(M, K, N, p.algo);
      *out = &(plans_[key] = p);
      return "";
    }
    // time each candidate (on the real operands; C is overwritten later)
    hipEvent_t e0, e1;
    (void)hipEventCreate(&e0);
    (void)hipEventCreate(&e1);
    float best = 1e30f;
    int bi = -1;
    const float alpha = 1.f, beta = 0.f;
    for (int a = 0; a < got; a++) {
      if (hipblasLtMatmul(h_, p.d, &alpha, W, p.la, B, p.lb, &beta, C, p.lc, C, p.lc, &res[a].algo,
                          ws_, wsz_, st) != HIPBLAS_STATUS_SUCCESS)
        continue;
      (void)hipEventRecord(e0, st);
      for (int r = 0; r < 3; r++)
        (void)hipblasLtMatmul(h_, p.d, &alpha, W, p.la, B, p.lb, &beta, C, p.lc, C, p.lc,
                              &res[a].algo, ws_, wsz_, st);
      (void)hipEventRecord(e1, st);
      (void)hipEventSynchronize(e1);
      float ms = 0.f;
      (void)hipEventElapsedTime(&ms, e0, e1);
      if (ms < best) {
        best = ms;
        bi = a;
      }
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (bi < 0) {
      destroy(p);
      return "every hipBLASLt candidate failed";
    }
    p.algo = res[bi].algo;
    note(M, K, N, p.algo);
    *out = &(plans_[key] = p);
    return "";
  }

  void note(int M, int K, int N, hipblasLtMatmulAlgo_t &algo) {
    if (!log_) return;
    fprintf(stderr, "[blas] M %d K %d N %d -> algorithm %d %s\n", M, K, N,
            hipblaslt_ext::getIndexFromAlgo(algo),
            hipblaslt_ext::getKernelNameFromAlgo(h_, algo).c_str());
  }
};

}  // namespace vx
