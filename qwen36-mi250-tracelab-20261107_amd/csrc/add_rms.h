// Residual add + zero-centred RMSNorm of token rows (the post-attention norm that feeds the
// MoE block): total = bf16(x + h), out = bf16(total * rsqrt(mean(total^2) + eps) * (1 + w)).
// Math of engine/fast/kernels.py:507-523 (_add_rms_kernel) and of Transformers'
// Qwen3_5MoeRMSNorm (modeling_qwen3_5_moe.py:801-815).
//
// One wave holds one row: lane l owns the 8 elements at c * 512 + 8 l of chunk c, so a row
// of H <= 512 HC elements is HC 16-byte loads per lane. The stand-alone kernel (k_add_rms)
// and the decode router's prologue both use add_rms_compute, so they give the same bits;
// the loads are separate so that a caller can issue other loads before the arithmetic.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "moe_common.h"
#include "route_sort_dev.h"

namespace moe {

constexpr int kAddRmsMaxChunks = 16;  // H <= 8192

// A row held as HC chunks of 8 bf16 per lane. Elements at or past H read as zero and are
// never stored; FULL: H == 512 HC, no element is out of range.
template <int HC, bool FULL = false>
__device__ __forceinline__ void load_row(const uint16_t* src, int H, int lane, uint4 (&v)[HC]) {
#pragma unroll
  for (int c = 0; c < HC; ++c) {
    const int e = c * 512 + lane * 8;
    v[c] = FULL || e < H ? ld16(src + e) : make_uint4(0u, 0u, 0u, 0u);
  }
}

// In place: tot (the x row) becomes total = bf16(x + h) when h is given (hv: the h row),
// and y the normalised row, with w (wv) the norm weight row.
template <int HC>
__device__ __forceinline__ void add_rms_compute(bool has_h, int H, float eps, uint4 (&tot)[HC],
                                                const uint4 (&hv)[HC], const uint4 (&wv)[HC],
                                                uint4 (&y)[HC]) {
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < HC; ++c) {
    uint32_t* t = &tot[c].x;
    const uint32_t* hh = &hv[c].x;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (has_h)  // the residual add rounds to bf16, as the bf16 tensor add does
        t[j] = pack_bf2_rne(bf_lo(t[j]) + bf_lo(hh[j]), bf_hi(t[j]) + bf_hi(hh[j]));
      const float lo = bf_lo(t[j]), hi = bf_hi(t[j]);
      ss = fmaf(lo, lo, ss);
      ss = fmaf(hi, hi, ss);
    }
  }
  ss = wave_sum(ss);
  const float r = rsqrtf(ss / (float)H + eps);
#pragma unroll
  for (int c = 0; c < HC; ++c) {
    const uint32_t* t = &tot[c].x;
    const uint32_t* ww = &wv[c].x;
    uint32_t* o = &y[c].x;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o[j] = pack_bf2_rne(bf_lo(t[j]) * r * (1.0f + bf_lo(ww[j])),
                          bf_hi(t[j]) * r * (1.0f + bf_hi(ww[j])));
  }
}

// Stores the in-range chunks of a row held as above.
template <int HC>
__device__ __forceinline__ void store_row(uint16_t* dst, int H, int lane, const uint4 (&v)[HC]) {
#pragma unroll
  for (int c = 0; c < HC; ++c) {
    const int e = c * 512 + lane * 8;
    if (e < H) st16(dst + e, v[c]);
  }
}

// total [T, H] (written only when h is given) and out [T, H]; H a multiple of 8, at most
// 512 * kAddRmsMaxChunks; rows 16-byte aligned.
hipError_t launch_add_rms(const uint16_t* x, const uint16_t* h, const uint16_t* w, int T, int H,
                          float eps, uint16_t* total, uint16_t* out, hipStream_t s);

}  // namespace moe
