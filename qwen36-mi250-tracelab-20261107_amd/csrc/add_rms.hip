// Stand-alone residual add + RMSNorm (add_rms.h): one wave per row, four rows per workgroup.
#include "add_rms.h"

namespace moe {
namespace {

template <int HC>
__global__ __launch_bounds__(256) void k_add_rms(const uint16_t* x, const uint16_t* h,
                                                 const uint16_t* w, int T, int H, float eps,
                                                 uint16_t* total, uint16_t* out) {
  const int lane = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= T) return;
  uint4 tot[HC], hv[HC], wv[HC], y[HC];
  load_row<HC>(x + row * H, H, lane, tot);
  if (h) load_row<HC>(h + row * H, H, lane, hv);
  load_row<HC>(w, H, lane, wv);
  add_rms_compute<HC>(h != nullptr, H, eps, tot, hv, wv, y);
  if (h) store_row<HC>(total + row * H, H, lane, tot);
  store_row<HC>(out + row * H, H, lane, y);
}

}  // namespace

hipError_t launch_add_rms(const uint16_t* x, const uint16_t* h, const uint16_t* w, int T, int H,
                          float eps, uint16_t* total, uint16_t* out, hipStream_t s) {
  if (T <= 0) return hipSuccess;
  if (H <= 0 || H % 8 || H > 512 * kAddRmsMaxChunks) return hipErrorInvalidValue;
  const dim3 grid((T + 3) / 4), block(256);
  const int hc = (H + 511) / 512;
#define L(HC)                                                                   \
  if (hc <= HC) {                                                               \
    hipLaunchKernelGGL((k_add_rms<HC>), grid, block, 0, s, x, h, w, T, H, eps, total, out); \
    return hipGetLastError();                                                   \
  }
  L(1) L(2) L(4) L(8) L(16)
#undef L
  return hipErrorInvalidValue;
}

}  // namespace moe
