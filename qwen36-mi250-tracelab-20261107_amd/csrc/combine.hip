// Weighted scatter-combine of the routed pairs plus the gated shared expert (a7, a10).
//
//   routed[t] = bf16( sum_j term(y[t*k + j], w[t, j]) )      fp32 sum in j order
//   term      = bf16(y * w)  (round_w: Transformers batched_mm, moe.py:165-171;
//                             engine/fast/kernels.py:163)
//             = y * w        (exact in fp32: engine/experts.py:53-57,
//                             engine/fast/moe_prefill.py:580-582)
//   moe[t]    = bf16(routed + bf16(bf16(sigmoid(bf16 seg_t)) * shared[t]))
//               (modeling_qwen3_5_moe.py:796-799; prefill_kernels.py:253-273)
//   out[t]    = bf16(residual[t] + moe[t])   when a residual is given (fused.py:641-692)
#include "moe_common.h"

namespace moe {

__global__ __launch_bounds__(256) void k_combine(
    const uint16_t* __restrict__ y, const uint16_t* __restrict__ w, int k,
    const uint16_t* __restrict__ ysh, const uint16_t* __restrict__ seg, long long ld_seg,
    const uint16_t* __restrict__ res, uint16_t* __restrict__ out, int T, int H, int round_w) {
  const int nb = (H / 8 + blockDim.x - 1) / blockDim.x;
  const int t = blockIdx.x / nb;
  const int c = ((blockIdx.x - t * nb) * blockDim.x + threadIdx.x) * 8;
  if (t >= T || c >= H) return;
  combine8(y, w, k, ysh, seg, ld_seg, res, out, t, H, c, round_w);
}

hipError_t launch_combine(const uint16_t* y, const uint16_t* w, int k, const uint16_t* ysh,
                          const uint16_t* seg, long long ld_seg, const uint16_t* res, uint16_t* out,
                          int T, int H, int round_w, hipStream_t s) {
  if (T <= 0) return hipSuccess;
  dim3 block(256);
  dim3 grid(((H / 8 + 255) / 256) * T);
  hipLaunchKernelGGL(k_combine, grid, block, 0, s, y, w, k, ysh, seg, ld_seg, res, out, T, H,
                     round_w);
  return hipGetLastError();
}

}  // namespace moe
