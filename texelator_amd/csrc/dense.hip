// Dense-scratch prefill: the GEMM half (hipBLASLt) and the bias epilogue.
//
// Reference: texelator_prefill_bf16_cublas (texelator/cuda/texelator_cuda.cu:937-990), backend 1
// and the fallback of backends 2-9 for shapes their kernels do not take: rows of the BC4 matrix
// are decoded tile_rows at a time into a dense 16-bit scratch matrix, one library GEMM per row
// tile writes Y[:, rows] directly (Y = X W^T, fp32 accumulation), and the bias is added afterwards
// with a second rounding (:982-989). Here the decode is launch_decode_rows, the scratch is the
// caller's workspace (no allocation on the call path) and the GEMM is hipBLASLt, the library
// torch-ROCm uses for its own bf16 GEMMs. hipBLASLt is opened with dlopen at the first dense
// call, so GEMV and tile-prefill callers never load it; in a process that already holds a copy
// (torch), the same soname resolves to that copy.
#include <dlfcn.h>
#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <tuple>

#include "elementwise.h"
#include "kernels.h"

namespace tx {

namespace {

struct BlasLt {
  decltype(&hipblasLtCreate) create = nullptr;
  decltype(&hipblasLtMatmulDescCreate) desc_create = nullptr;
  decltype(&hipblasLtMatmulDescSetAttribute) desc_set = nullptr;
  decltype(&hipblasLtMatrixLayoutCreate) layout_create = nullptr;
  decltype(&hipblasLtMatmulPreferenceCreate) pref_create = nullptr;
  decltype(&hipblasLtMatmulPreferenceSetAttribute) pref_set = nullptr;
  decltype(&hipblasLtMatmulAlgoGetHeuristic) heuristic = nullptr;
  decltype(&hipblasLtMatmul) matmul = nullptr;
  decltype(&hipblasLtMatmulDescDestroy) desc_destroy = nullptr;
  decltype(&hipblasLtMatrixLayoutDestroy) layout_destroy = nullptr;
  decltype(&hipblasLtMatmulPreferenceDestroy) pref_destroy = nullptr;
  std::string error;  // why the library could not be opened, if it could not
};

const BlasLt &blaslt() {
  static const BlasLt api = [] {
    BlasLt a;
    void *lib = dlopen("libhipblaslt.so.1", RTLD_NOW | RTLD_LOCAL);
    if (!lib) lib = dlopen("libhipblaslt.so", RTLD_NOW | RTLD_LOCAL);
    if (!lib) {
      const char *why = dlerror();
      a.error = std::string("cannot open hipBLASLt (libhipblaslt.so.1): ") + (why ? why : "unknown error");
      return a;
    }
    auto sym = [&](auto &fn, const char *name) {
      fn = reinterpret_cast<std::remove_reference_t<decltype(fn)>>(dlsym(lib, name));
      if (!fn && a.error.empty()) a.error = std::string("hipBLASLt lacks ") + name;
    };
    sym(a.create, "hipblasLtCreate");
    sym(a.desc_create, "hipblasLtMatmulDescCreate");
    sym(a.desc_set, "hipblasLtMatmulDescSetAttribute");
    sym(a.layout_create, "hipblasLtMatrixLayoutCreate");
    sym(a.pref_create, "hipblasLtMatmulPreferenceCreate");
    sym(a.pref_set, "hipblasLtMatmulPreferenceSetAttribute");
    sym(a.heuristic, "hipblasLtMatmulAlgoGetHeuristic");
    sym(a.matmul, "hipblasLtMatmul");
    sym(a.desc_destroy, "hipblasLtMatmulDescDestroy");
    sym(a.layout_destroy, "hipblasLtMatrixLayoutDestroy");
    sym(a.pref_destroy, "hipblasLtMatmulPreferenceDestroy");
    return a;
  }();
  return api;
}

// A prepared GEMM for one (device, dtype, rows, tokens, K, ldy): descriptors and the first
// algorithm the heuristic offers whose state is success and whose workspace fits the
// kDenseGemmWorkspace bytes the caller provides (split-K algorithms of long-K, few-row shapes use
// one). At most kMaxPlans are kept (a server with many prompt lengths would otherwise add one per
// length); the least recently used is destroyed to make room. Plans are created, used and
// destroyed under g_mutex, so no call ever holds a destroyed descriptor.
struct Plan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  uint64_t last_use = 0;
};

constexpr size_t kMaxPlans = 64;

void destroy_plan(const BlasLt &api, Plan &plan) {
  if (plan.desc) api.desc_destroy(plan.desc);
  if (plan.a) api.layout_destroy(plan.a);
  if (plan.b) api.layout_destroy(plan.b);
  if (plan.d) api.layout_destroy(plan.d);
  plan = Plan{};
}

std::mutex g_mutex;
std::map<int, hipblasLtHandle_t> g_handles;
std::map<std::tuple<int, bool, int, int64_t, int, int64_t>, Plan> g_plans;
uint64_t g_use_clock = 0;

std::string status_text(const char *what, hipblasStatus_t status) {
  return std::string("hipBLASLt ") + what + " failed (status " + std::to_string((int)status) + ")";
}

// y = round(y + bias) per element; one thread per output element.
template <bool F16>
__global__ __launch_bounds__(256) void add_bias_kernel(uint16_t *y, const uint16_t *bias, int64_t n, int M) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float v = half_bits_to_float<F16>(y[i]) + half_bits_to_float<F16>(bias[i % M]);
  if constexpr (F16) y[i] = __builtin_bit_cast(uint16_t, (_Float16)v);
  else y[i] = to_bf(v);
}

}  // namespace

bool dense_gemm(int device, bool f16, int rows, int64_t tokens, int K, const void *w, const void *x, void *y,
                int64_t ldy, void *gemm_workspace, hipStream_t stream, std::string &error) {
  const BlasLt &api = blaslt();
  if (!api.error.empty()) {
    error = api.error;
    return false;
  }
  std::lock_guard<std::mutex> lock(g_mutex);
  hipblasLtHandle_t handle = nullptr;
  auto found = g_handles.find(device);
  if (found == g_handles.end()) {
    const hipblasStatus_t s = api.create(&handle);
    if (s != HIPBLAS_STATUS_SUCCESS) {
      error = status_text("handle creation", s);
      return false;
    }
    g_handles[device] = handle;
  } else {
    handle = found->second;
  }
  const auto key = std::make_tuple(device, f16, rows, tokens, K, ldy);
  auto cached = g_plans.find(key);
  if (cached == g_plans.end()) {
    // Column-major view of the row-major operands: D (rows x tokens, ld ldy) =
    // op(A) * B with A = W^T (K x rows, ld K) transposed and B = X^T (K x tokens, ld K).
    Plan plan;
    const hipDataType type = f16 ? HIP_R_16F : HIP_R_16BF;
    hipblasStatus_t s = api.desc_create(&plan.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F);
    const int32_t trans_a = HIPBLAS_OP_T, trans_b = HIPBLAS_OP_N;
    if (s == HIPBLAS_STATUS_SUCCESS) s = api.desc_set(plan.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &trans_a, sizeof(trans_a));
    if (s == HIPBLAS_STATUS_SUCCESS) s = api.desc_set(plan.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &trans_b, sizeof(trans_b));
    if (s == HIPBLAS_STATUS_SUCCESS) s = api.layout_create(&plan.a, type, (uint64_t)K, (uint64_t)rows, K);
    if (s == HIPBLAS_STATUS_SUCCESS) s = api.layout_create(&plan.b, type, (uint64_t)K, (uint64_t)tokens, K);
    if (s == HIPBLAS_STATUS_SUCCESS) s = api.layout_create(&plan.d, type, (uint64_t)rows, (uint64_t)tokens, ldy);
    if (s != HIPBLAS_STATUS_SUCCESS) {
      destroy_plan(api, plan);
      error = status_text("descriptor creation", s);
      return false;
    }
    hipblasLtMatmulPreference_t pref = nullptr;
    s = api.pref_create(&pref);
    const uint64_t max_workspace = kDenseGemmWorkspace;
    if (s == HIPBLAS_STATUS_SUCCESS)
      s = api.pref_set(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &max_workspace, sizeof(max_workspace));
    constexpr int kAsk = 8;
    hipblasLtMatmulHeuristicResult_t results[kAsk]{};
    int count = 0;
    if (s == HIPBLAS_STATUS_SUCCESS)
      s = api.heuristic(handle, plan.desc, plan.a, plan.b, plan.d, plan.d, pref, kAsk, results, &count);
    if (pref) api.pref_destroy(pref);
    if (s != HIPBLAS_STATUS_SUCCESS) {
      destroy_plan(api, plan);
      error = status_text("heuristic", s);
      return false;
    }
    int pick = -1;
    for (int i = 0; i < std::min(count, kAsk) && pick < 0; ++i)
      if (results[i].state == HIPBLAS_STATUS_SUCCESS && results[i].workspaceSize <= kDenseGemmWorkspace) pick = i;
    if (pick < 0) {
      destroy_plan(api, plan);
      error = "hipBLASLt offers no algorithm for this shape within " + std::to_string(kDenseGemmWorkspace) +
              " bytes of workspace";
      return false;
    }
    plan.algo = results[pick].algo;
    if (g_plans.size() >= kMaxPlans) {
      auto oldest = g_plans.begin();
      for (auto it = g_plans.begin(); it != g_plans.end(); ++it)
        if (it->second.last_use < oldest->second.last_use) oldest = it;
      destroy_plan(api, oldest->second);
      g_plans.erase(oldest);
    }
    cached = g_plans.emplace(key, plan).first;
  }
  Plan &plan = cached->second;
  plan.last_use = ++g_use_clock;
  const float alpha = 1.f, beta = 0.f;
  const hipblasStatus_t s = api.matmul(handle, plan.desc, &alpha, w, plan.a, x, plan.b, &beta, y, plan.d, y, plan.d,
                                       &plan.algo, gemm_workspace, kDenseGemmWorkspace, stream);
  if (s != HIPBLAS_STATUS_SUCCESS) {
    error = status_text("matmul", s);
    return false;
  }
  return true;
}

hipError_t launch_add_bias(void *y, const void *bias, int64_t tokens, int M, bool f16, hipStream_t stream) {
  const int64_t n = tokens * M;
  const dim3 grid((unsigned)((n + 255) / 256));
  if (f16)
    hipLaunchKernelGGL(add_bias_kernel<true>, grid, dim3(256), 0, stream, static_cast<uint16_t *>(y),
                       static_cast<const uint16_t *>(bias), n, M);
  else
    hipLaunchKernelGGL(add_bias_kernel<false>, grid, dim3(256), 0, stream, static_cast<uint16_t *>(y),
                       static_cast<const uint16_t *>(bias), n, M);
  return hipGetLastError();
}

}  // namespace tx
