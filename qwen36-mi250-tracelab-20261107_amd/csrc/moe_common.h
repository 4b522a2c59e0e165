// Shared device helpers for the MI355X (gfx950) MoE kernels.
//
// Numerics follow the rounding points of the Transformers / engine torch path:
// every projection output, activation and product is rounded to bf16 with
// round-to-nearest-even, exactly as a bf16 torch tensor op rounds its fp32 result.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moe {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// fp32 -> bf16 bits, round to nearest even (NaN kept quiet). Bit-identical to
// torch's float->bfloat16 conversion.
__device__ __forceinline__ uint16_t f2bf_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float bf_bits2f(uint32_t b) { return __uint_as_float(b << 16); }
// fp32 rounded to bf16 and widened back to fp32.
__device__ __forceinline__ float rbf(float f) { return bf_bits2f(f2bf_bits(f)); }

// Low / high bf16 of a packed 32-bit word, as fp32.
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  return (uint32_t)f2bf_bits(lo) | ((uint32_t)f2bf_bits(hi) << 16);
}

// torch's sigmoid / silu on a bf16 input evaluate in fp32; the caller rounds.
__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float siluf_(float x) { return x / (1.0f + expf(-x)); }

// 16-byte global load/store helpers (one global_load_dwordx4 per lane).
__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ void st16(void* p, uint4 v) { *reinterpret_cast<uint4*>(p) = v; }

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) {
  return __builtin_bit_cast(bf16x8_t, v);
}

// 16 OCP e4m3fn bytes -> two bf16x8 operands (exact: every e4m3 value is a bf16 value).
// gfx950's scaled conversion with scale 1.0 turns two e4m3 bytes into two bf16 in one step.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
template <bool HI>
__device__ __forceinline__ uint32_t fp8x2_to_bf16x2(uint32_t w) {
  bf16x2_t r = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI);
  return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ void fp8x16_to_bf16(uint4 q, uint4& lo, uint4& hi) {
  lo.x = fp8x2_to_bf16x2<false>(q.x);
  lo.y = fp8x2_to_bf16x2<true>(q.x);
  lo.z = fp8x2_to_bf16x2<false>(q.y);
  lo.w = fp8x2_to_bf16x2<true>(q.y);
  hi.x = fp8x2_to_bf16x2<false>(q.z);
  hi.y = fp8x2_to_bf16x2<true>(q.z);
  hi.z = fp8x2_to_bf16x2<false>(q.w);
  hi.w = fp8x2_to_bf16x2<true>(q.w);
}

__device__ __forceinline__ f32x4_t mfma16x16x32(uint4 a, uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// Tile table layout (shared with the host): for max_tiles MT,
//   table[t] = expert, table[MT + t] = first sorted row, table[2 MT + t] = row end,
//   table[3 MT] = number of tiles.
struct TileRef {
  int expert, row0, row1;
};

}  // namespace moe
