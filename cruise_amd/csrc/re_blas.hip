// Batched-prefill projections on hipBLASLt (bf16 in and out, fp32
// accumulation).  The prefill GEMMs are plain large GEMMs (M = prompt tokens
// of the batch, N x K a weight matrix), the case AMD's tuned library is
// made for; the decode step keeps its hand-written weight-streaming kernels.
//
// out[M, N] = T(A[M, K] W[N, K]^T (+ bias[N])), row-major bf16, computed as the
// column-major TN product D[N, M] = W^T' A' that hipBLASLt plans: the bias
// is added in fp32 before the single rounding (F.linear with bias,
// g4a_linear_t_bias.py:18-21).  The residual projections (o-proj, down) go
// through a T-rounded product and then h = T(h + y) (k_pf_residual): the
// reference's rounding points (batched_decoder_step.py:380-386, 399-403).
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <tuple>

#include "re_device.h"
#include "re_layout.h"

namespace re {

struct PrefillBlas {
  hipblasLtHandle_t handle = nullptr;
  void* workspace = nullptr;
  size_t workspace_bytes = 0;
  // heuristic's first algorithm per (M, N, K, bias, lda, ldw, ldo)
  std::map<std::tuple<int, int, int, int, long long, long long, long long>, hipblasLtMatmulAlgo_t> algos;
};

namespace {

constexpr size_t kWorkspaceBytes = 64u << 20;

// h = T(h + y) over rows of N elements (both bf16, row strides ldh and ldy).
__global__ void __launch_bounds__(256) k_pf_residual(bf16_t* h, const bf16_t* y, long long rows, int N, long long ldh,
                                                      long long ldy) {
  const int per_row = N / 8;
  const long long n = rows * per_row;
  for (long long i = blockIdx.x * 256LL + threadIdx.x; i < n; i += (long long)gridDim.x * 256) {
    const long long r = i / per_row;
    const int c = static_cast<int>(i - r * per_row) * 8;
    Vec8<bf16_t>* hp = reinterpret_cast<Vec8<bf16_t>*>(h + r * ldh + c);
    const Vec8<bf16_t> hv = *hp;
    const Vec8<bf16_t> yv = Vec8<bf16_t>::load(y + r * ldy + c);
    float out[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = hv.get(e) + yv.get(e);
    *hp = Vec8<bf16_t>::from_floats(out);
  }
}

struct Desc {
  hipblasLtMatmulDesc_t op = nullptr;
  hipblasLtMatrixLayout_t w = nullptr, a = nullptr, d = nullptr;
  ~Desc() {
    if (d) hipblasLtMatrixLayoutDestroy(d);
    if (a) hipblasLtMatrixLayoutDestroy(a);
    if (w) hipblasLtMatrixLayoutDestroy(w);
    if (op) hipblasLtMatmulDescDestroy(op);
  }
};

bool make_desc(Desc& ds, const GemmArgs& g) {
  if (hipblasLtMatmulDescCreate(&ds.op, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS) return false;
  const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  if (hipblasLtMatmulDescSetAttribute(ds.op, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatmulDescSetAttribute(ds.op, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) != HIPBLAS_STATUS_SUCCESS)
    return false;
  if (g.bias != nullptr) {
    const hipblasLtEpilogue_t ep = HIPBLASLT_EPILOGUE_BIAS;
    const void* bp = g.bias;
    const int32_t bt = HIP_R_16BF;
    if (hipblasLtMatmulDescSetAttribute(ds.op, HIPBLASLT_MATMUL_DESC_EPILOGUE, &ep, sizeof(ep)) !=
            HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatmulDescSetAttribute(ds.op, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bp, sizeof(bp)) !=
            HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatmulDescSetAttribute(ds.op, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof(bt)) !=
            HIPBLAS_STATUS_SUCCESS)
      return false;
  }
  // W [N, K] row-major is the column-major K x N matrix (op T); A [M, K] the
  // column-major K x M matrix; out [M, N] the column-major N x M matrix.
  return hipblasLtMatrixLayoutCreate(&ds.w, HIP_R_16BF, g.K, g.N, g.ldw) == HIPBLAS_STATUS_SUCCESS &&
         hipblasLtMatrixLayoutCreate(&ds.a, HIP_R_16BF, g.K, g.M, g.lda) == HIPBLAS_STATUS_SUCCESS &&
         hipblasLtMatrixLayoutCreate(&ds.d, HIP_R_16BF, g.N, g.M, g.ldo) == HIPBLAS_STATUS_SUCCESS;
}

}  // namespace

PrefillBlas* prefill_blas_create() {
  PrefillBlas* b = new PrefillBlas();
  if (hipblasLtCreate(&b->handle) != HIPBLAS_STATUS_SUCCESS) {
    b->handle = nullptr;
    prefill_blas_destroy(b);
    return nullptr;
  }
  if (hipMalloc(&b->workspace, kWorkspaceBytes) != hipSuccess) {
    b->workspace = nullptr;
    prefill_blas_destroy(b);
    return nullptr;
  }
  b->workspace_bytes = kWorkspaceBytes;
  return b;
}

void prefill_blas_destroy(PrefillBlas* b) {
  if (b == nullptr) return;
  if (b->workspace) (void)hipFree(b->workspace);
  if (b->handle) hipblasLtDestroy(b->handle);
  delete b;
}

// out = T(A W^T (+ bias)); false when hipBLASLt has no plan for the shape
// (the caller then runs its own kernel).
bool prefill_blas_gemm(PrefillBlas* b, const GemmArgs& g, hipStream_t stream) {
  if (b == nullptr || g.M <= 0 || g.N <= 0 || g.K <= 0) return false;
  Desc ds;
  if (!make_desc(ds, g)) return false;
  const auto key = std::make_tuple(g.M, g.N, g.K, g.bias != nullptr ? 1 : 0, g.lda, g.ldw, g.ldo);
  auto it = b->algos.find(key);
  if (it == b->algos.end()) {
    hipblasLtMatmulPreference_t pref = nullptr;
    if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) return false;
    const uint64_t ws = b->workspace_bytes;
    hipblasLtMatmulHeuristicResult_t res{};
    int n = 0;
    const bool found =
        hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws)) ==
            HIPBLAS_STATUS_SUCCESS &&
        hipblasLtMatmulAlgoGetHeuristic(b->handle, ds.op, ds.w, ds.a, ds.d, ds.d, pref, 1, &res, &n) ==
            HIPBLAS_STATUS_SUCCESS &&
        n > 0 && res.state == HIPBLAS_STATUS_SUCCESS;
    hipblasLtMatmulPreferenceDestroy(pref);
    if (!found) return false;
    if (b->algos.size() >= 256) b->algos.clear();  // prompt sizes vary; keep the cache small
    it = b->algos.emplace(key, res.algo).first;
  }
  const float alpha = 1.f, beta = 0.f;
  return hipblasLtMatmul(b->handle, ds.op, &alpha, g.W, ds.w, g.A, ds.a, &beta, g.out, ds.d, g.out, ds.d, &it->second,
                         b->workspace, b->workspace_bytes, stream) == HIPBLAS_STATUS_SUCCESS;
}

hipError_t launch_prefill_residual(void* h, const void* y, long long rows, int N, long long ldh, long long ldy,
                                   hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  if (N % 8 != 0 || ldh % 8 != 0 || ldy % 8 != 0) return hipErrorInvalidValue;
  const long long n = rows * (N / 8);
  const int blocks = static_cast<int>(std::min<long long>((n + 255) / 256, 16384));
  k_pf_residual<<<blocks, 256, 0, stream>>>(static_cast<bf16_t*>(h), static_cast<const bf16_t*>(y), rows, N, ldh, ldy);
  return hipGetLastError();
}

}  // namespace re
