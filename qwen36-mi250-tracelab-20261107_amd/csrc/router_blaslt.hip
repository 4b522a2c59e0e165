// Router logits of prefill-sized batches through hipBLASLt (subsystem a1).
//
// logits [T, n_pack] = bf16(x [T, H] . w_pack [n_pack, H]^T) with fp32 accumulation is a
// plain dense GEMM (the reference computes it with F.linear, modeling_qwen3_5_moe.py:768-769
// / engine/fast/model.py:1159, i.e. hipBLASLt under torch): above a few hundred tokens the
// library's tuned kernels beat the expert GEMM's identity tiles (measured 15 µs against 38 µs
// at 4096 tokens). Column-major view: C [n_pack, T] = op(A) [n_pack, H] . B [H, T] with A =
// w_pack stored [H, n_pack] (transposed), B = x stored [H, T], C = logits stored [n_pack, T].
//
// One handle per device and one cached plan (descriptors + heuristic algorithm) per shape;
// no workspace, so a call allocates nothing and can be captured in a HIP graph.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

namespace moe {

namespace {

struct Plan {
  hipblasLtMatmulDesc_t op = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  bool ok = false;
};

struct DeviceState {
  hipblasLtHandle_t handle = nullptr;
  std::map<std::tuple<int, int, int>, Plan> plans;
};

std::mutex g_mu;
DeviceState g_dev[64];

Plan* plan_for(int dev, int T, int H, int n_pack) {
  DeviceState& ds = g_dev[dev];
  if (!ds.handle && hipblasLtCreate(&ds.handle) != HIPBLAS_STATUS_SUCCESS) {
    ds.handle = nullptr;
    return nullptr;
  }
  Plan& p = ds.plans[std::make_tuple(T, H, n_pack)];
  if (p.ok) return &p;
  if (p.op) return nullptr;  // tried and failed before
  if (hipblasLtMatmulDescCreate(&p.op, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS)
    return nullptr;
  hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta));
  hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb));
  if (hipblasLtMatrixLayoutCreate(&p.a, HIP_R_16BF, H, n_pack, H) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatrixLayoutCreate(&p.b, HIP_R_16BF, H, T, H) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatrixLayoutCreate(&p.c, HIP_R_16BF, n_pack, T, n_pack) != HIPBLAS_STATUS_SUCCESS)
    return nullptr;
  hipblasLtMatmulPreference_t pref = nullptr;
  if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) return nullptr;
  uint64_t ws = 0;
  hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws,
                                        sizeof(ws));
  hipblasLtMatmulHeuristicResult_t res{};
  int count = 0;
  const hipblasStatus_t st = hipblasLtMatmulAlgoGetHeuristic(ds.handle, p.op, p.a, p.b, p.c, p.c,
                                                             pref, 1, &res, &count);
  hipblasLtMatmulPreferenceDestroy(pref);
  if (st != HIPBLAS_STATUS_SUCCESS || count < 1) return nullptr;
  p.algo = res.algo;
  p.ok = true;
  return &p;
}

}  // namespace

// hipErrorInvalidValue: no hipBLASLt plan for this shape (the caller uses its own kernel).
hipError_t launch_router_blaslt(const void* x, int T, int H, const void* w_pack, int n_pack,
                                void* logits, hipStream_t st) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return hipErrorInvalidValue;
  Plan* p;
  hipblasLtHandle_t h;
  {
    std::lock_guard<std::mutex> lock(g_mu);
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess) return hipErrorInvalidValue;
    const bool capturing = cs != hipStreamCaptureStatusNone;
    // plans are made outside capture only (the heuristic query is not a stream operation,
    // but handle creation may allocate)
    if (capturing) {
      DeviceState& ds = g_dev[dev];
      auto it = ds.plans.find(std::make_tuple(T, H, n_pack));
      if (!ds.handle || it == ds.plans.end() || !it->second.ok) return hipErrorInvalidValue;
      p = &it->second;
    } else {
      p = plan_for(dev, T, H, n_pack);
      if (!p) return hipErrorInvalidValue;
    }
    h = g_dev[dev].handle;
  }
  const float alpha = 1.0f, beta = 0.0f;
  const hipblasStatus_t s = hipblasLtMatmul(h, p->op, &alpha, w_pack, p->a, x, p->b, &beta, logits,
                                            p->c, logits, p->c, &p->algo, nullptr, 0, st);
  return s == HIPBLAS_STATUS_SUCCESS ? hipSuccess : hipErrorLaunchFailure;
}

}  // namespace moe
