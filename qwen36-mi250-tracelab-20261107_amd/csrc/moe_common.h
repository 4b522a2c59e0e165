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

// Comparison switches of the launch path (MOE_DECODE, MOE_DECODE_DOWN, MOE_DECODE_GU_BLOCKS,
// MOE_MIXED, MOE_PREFILL_SIDE, MOE_PREFILL_SHARED_FIRST,
// MOE_GEMM_SHARED_FIRST): each selects a variant that the
// GPU tests compare with the default. They are read from the environment once per process
// and again by moe_reload_tuning(), never per launch.
enum Knob {
  kKnobDecode,
  kKnobDecodeDown,
  kKnobDecodeGuBlocks,
  kKnobMixed,
  kKnobPrefillSide,
  kKnobPrefillSharedFirst,
  kKnobGemmSharedFirst,
  kKnobCount
};
// The switch's value, or nullptr when it is unset (host code).
const char* knob(Knob k);

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

// Two fp32 -> packed bf16 with gfx950's v_cvt_pk_bf16_f32 (round to nearest even, as
// f2bf_bits for every non-NaN input): one instruction where f2bf_bits takes several.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf2_rne(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// torch's sigmoid / silu on a bf16 input evaluate in fp32; the caller rounds.
__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float siluf_(float x) { return x / (1.0f + expf(-x)); }

// 16-byte global load/store helpers (one global_load_dwordx4 per lane).
__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ void st16(void* p, uint4 v) { *reinterpret_cast<uint4*>(p) = v; }
// Streaming (non-temporal) loads for weights read once per launch: they need not displace
// the L2 lines of data that is reused (token rows, activations).
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 ld16_stream(const void* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ld8_stream(const void* p) {
  const u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
  return make_uint2(v.x, v.y);
}

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

// Weighted combine of 8 consecutive columns c..c+7 of token t (see combine.hip):
//   bf16(bf16(sum_j term(y[t*k+j], w[t*k+j])) + bf16(bf16(sigmoid(seg_t)) * ysh[t]))
//   (+ residual), term = bf16(y*w) when round_w else y*w (exact in fp32).
__device__ __forceinline__ void combine8(const uint16_t* __restrict__ y,
                                         const uint16_t* __restrict__ w, int k,
                                         const uint16_t* __restrict__ ysh,
                                         const uint16_t* __restrict__ seg, long long ld_seg,
                                         const uint16_t* __restrict__ res,
                                         uint16_t* __restrict__ out, int t, int H, int c,
                                         int round_w) {
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;
  // Pairs in groups of 8 whose loads are all issued before the first is used: one memory
  // round trip per group instead of one per pair.
  for (int j0 = 0; j0 < k; j0 += 8) {
    uint4 v[8];
    float wj[8];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const long long p = (long long)t * k + min(j0 + jj, k - 1);
      v[jj] = ld16(y + p * H + c);
      wj[jj] = bf_bits2f(w[p]);
    }
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      if (j0 + jj >= k) break;
      uint32_t u[4] = {v[jj].x, v[jj].y, v[jj].z, v[jj].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float a = bf_lo(u[i]) * wj[jj], b = bf_hi(u[i]) * wj[jj];
        if (round_w) {
          a = rbf(a);
          b = rbf(b);
        }
        acc[2 * i] += a;
        acc[2 * i + 1] += b;
      }
    }
  }
  float o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = rbf(acc[i]);
  if (ysh) {
    float g = rbf(sigmoidf_(bf_bits2f(seg[(long long)t * ld_seg])));
    uint4 v = ld16(ysh + (long long)t * H + c);
    uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = rbf(o[2 * i] + rbf(g * bf_lo(u[i])));
      o[2 * i + 1] = rbf(o[2 * i + 1] + rbf(g * bf_hi(u[i])));
    }
  }
  if (res) {
    uint4 v = ld16(res + (long long)t * H + c);
    uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = o[2 * i] + bf_lo(u[i]);
      o[2 * i + 1] = o[2 * i + 1] + bf_hi(u[i]);
    }
  }
  uint4 r;
  r.x = pack_bf2(o[0], o[1]);
  r.y = pack_bf2(o[2], o[3]);
  r.z = pack_bf2(o[4], o[5]);
  r.w = pack_bf2(o[6], o[7]);
  st16(out + (long long)t * H + c, r);
}

// Tile table layout (shared with the host): for max_tiles MT,
//   table[t] = expert, table[MT + t] = first sorted row, table[2 MT + t] = row end,
//   table[3 MT] = number of tiles.
struct TileRef {
  int expert, row0, row1;
};

}  // namespace moe
