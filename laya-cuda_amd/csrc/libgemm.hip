// Plain projections through hipBLASLt: out[M][N] = x[M][K] W[N][K]^T (+ fp32 bias before the single
// rounding to 16 bits), the batched slots' attention-output and FFN-down projections.  These are the
// only GEMMs here without a fused epilogue of their own (head-major QKV scatter with RoPE, GELU,
// GeGLU), and on the 64K-row problems hipBLASLt's kernels ran 14-22% faster than the MFMA tiles of
// gemm.hip in isolated launches; the runtime times both on each new batched slot and keeps the
// faster one, so this file only describes the problem and runs the candidates the library offers.
//
// hipBLASLt is column-major: the row-major out[M][N] is the column-major N x M matrix
// D = op(A) B with A = W seen as the column-major K x N matrix (op = transpose) and B = x seen as
// the column-major K x M matrix.  The bias (N fp32 values) is broadcast along D's columns, i.e.
// added to every output row, in the fp32 accumulator before the conversion to 16 bits.
#include <hipblaslt/hipblaslt.h>

#include "kernels.hpp"

namespace laya {

struct LibGemm {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
  hipblasLtMatmulAlgo_t algo[kLibCandidates];
  size_t ws[kLibCandidates] = {};
  int candidates = 0, chosen = -1;
  bool bias = false;
};

void* lib_handle_create() {
  hipblasLtHandle_t h = nullptr;
  return hipblasLtCreate(&h) == HIPBLAS_STATUS_SUCCESS ? h : nullptr;
}

void lib_handle_destroy(void* handle) {
  if (handle) (void)hipblasLtDestroy(static_cast<hipblasLtHandle_t>(handle));
}

void lib_gemm_destroy(LibGemm* g) {
  if (!g) return;
  if (g->desc) (void)hipblasLtMatmulDescDestroy(g->desc);
  if (g->a) (void)hipblasLtMatrixLayoutDestroy(g->a);
  if (g->b) (void)hipblasLtMatrixLayoutDestroy(g->b);
  if (g->d) (void)hipblasLtMatrixLayoutDestroy(g->d);
  delete g;
}

LibGemm* lib_gemm_plan(void* handle, DType t, int M, int N, int K, bool bias, size_t max_ws) {
  if (!handle || M <= 0 || N <= 0 || K <= 0) return nullptr;
  LibGemm* g = new LibGemm();
  g->bias = bias;
  const hipDataType dt = t == DType::F16 ? HIP_R_16F : HIP_R_16BF;
  bool ok = hipblasLtMatmulDescCreate(&g->desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS;
  const int32_t op_t = HIPBLAS_OP_T, op_n = HIPBLAS_OP_N;
  const uint32_t epilogue = bias ? HIPBLASLT_EPILOGUE_BIAS : HIPBLASLT_EPILOGUE_DEFAULT;
  const int32_t bias_type = HIP_R_32F;
  ok = ok && hipblasLtMatmulDescSetAttribute(g->desc, HIPBLASLT_MATMUL_DESC_TRANSA, &op_t, sizeof(op_t)) ==
                 HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatmulDescSetAttribute(g->desc, HIPBLASLT_MATMUL_DESC_TRANSB, &op_n, sizeof(op_n)) ==
                 HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatmulDescSetAttribute(g->desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epilogue,
                                             sizeof(epilogue)) == HIPBLAS_STATUS_SUCCESS;
  if (bias)
    ok = ok && hipblasLtMatmulDescSetAttribute(g->desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bias_type,
                                               sizeof(bias_type)) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatrixLayoutCreate(&g->a, dt, K, N, K) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatrixLayoutCreate(&g->b, dt, K, M, K) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatrixLayoutCreate(&g->d, dt, N, M, N) == HIPBLAS_STATUS_SUCCESS;
  hipblasLtMatmulPreference_t pref = nullptr;
  ok = ok && hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS;
  const uint64_t ws = max_ws;
  ok = ok && hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws,
                                                   sizeof(ws)) == HIPBLAS_STATUS_SUCCESS;
  hipblasLtMatmulHeuristicResult_t found[kLibCandidates];
  int returned = 0;
  ok = ok && hipblasLtMatmulAlgoGetHeuristic(static_cast<hipblasLtHandle_t>(handle), g->desc, g->a, g->b, g->d,
                                             g->d, pref, kLibCandidates, found, &returned) == HIPBLAS_STATUS_SUCCESS;
  if (pref) (void)hipblasLtMatmulPreferenceDestroy(pref);
  for (int i = 0; ok && i < returned; ++i) {
    if (found[i].state != HIPBLAS_STATUS_SUCCESS || found[i].workspaceSize > max_ws) continue;
    g->algo[g->candidates] = found[i].algo;
    g->ws[g->candidates] = found[i].workspaceSize;
    ++g->candidates;
  }
  if (!ok || g->candidates == 0) {
    lib_gemm_destroy(g);
    return nullptr;
  }
  return g;
}

int lib_gemm_candidates(const LibGemm* g) { return g ? g->candidates : 0; }
size_t lib_gemm_workspace(const LibGemm* g, int candidate) { return g->ws[candidate]; }
int lib_gemm_chosen(const LibGemm* g) { return g ? g->chosen : -1; }
void lib_gemm_choose(LibGemm* g, int candidate) { g->chosen = candidate; }

bool lib_gemm_run(void* handle, LibGemm* g, int candidate, const void* w, const void* x, const float* bias,
                  void* out, void* ws, hipStream_t stream) {
  if (candidate < 0 || candidate >= g->candidates) return false;
  if (g->bias && hipblasLtMatmulDescSetAttribute(g->desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias,
                                                 sizeof(bias)) != HIPBLAS_STATUS_SUCCESS)
    return false;
  const float one = 1.f, zero = 0.f;
  return hipblasLtMatmul(static_cast<hipblasLtHandle_t>(handle), g->desc, &one, w, g->a, x, g->b, &zero, out, g->d,
                         out, g->d, &g->algo[candidate], ws, g->ws[candidate], stream) == HIPBLAS_STATUS_SUCCESS;
}

}  // namespace laya
