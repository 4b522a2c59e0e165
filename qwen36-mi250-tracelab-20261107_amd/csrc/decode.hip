// Decode-sized MoE block (T <= 4 tokens) on gfx950 in three launches
// (subsystems a1, a2, a4, a5, a6, a7, a10, a12 for decode batches).
//
// Same results contract as the tiled path (router -> route/sort -> grouped gate_up ->
// grouped down -> combine; engine/fast/fused.py:887-932, engine/fast/kernels.py:88-164,
// engine/fast/model.py:1139-1179), with the work regrouped for a handful of tokens, where
// every weight byte is used by at most four tokens and the block is bound by HBM latency
// and bandwidth rather than by any arithmetic:
//
//   K1 k_dec_router   one wave per router row (logits[t, n] = bf16(x_t . Wpack[n])) and one
//                     wave per shared-expert gate/up row pair (act_sh = SwiGLU). The shared
//                     expert does not depend on the routing, so its 4 MiB stream overlaps the
//                     router's HBM round trip instead of following it. Optionally it
//                     first computes the layer's post-attention add + RMSNorm of the token
//                     rows itself (every wave already reads whole rows), which removes that
//                     launch from a decode layer.
//   K2 k_dec_gate_up  every workgroup recomputes the softmax / top-k of the T tokens from the
//                     logits (a few hundred cycles; it replaces the route + sort launch),
//                     numbers the distinct experts in first-use order, takes one of them and
//                     four gate/up row pairs of it, and writes act[pair, n]. For one token
//                     the weight rows are requested as soon as the selection has reached the
//                     workgroup's expert, and the rest of the routing overlaps them.
//   K3 k_dec_down     one wave per hidden row n: y_p = bf16(act_p . Wd[e_p, n]) for every
//                     pair, the shared expert's row, and the combine of those values in the
//                     routing order j, gated shared term and residual, written straight to out.
//
// Every projection is a dot product over a whole weight row: lane l holds elements
// [512 c + 8 l, 512 c + 8 l + 8) of chunk c, so one load instruction reads 1 KiB (bf16) or
// 512 B (fp8) of one row contiguously; partial sums are reduced with DPP in a fixed order.
// Rounding points are those of the tiled kernels (rbf after each projection, SwiGLU as
// bf16(bf16(silu(bf16 g)) * bf16 u), combine terms bf16(w * y) under round_w).
#include <stdlib.h>

#include "moe_common.h"
#include "route_sort_dev.h"
#include "add_rms.h"
#include "lds_dma.h"
#include "decode.h"

namespace moe {

namespace {

constexpr int kDecThreads = 256;  // K3 (several tokens): four waves, one row each
constexpr int kGuWaves = 4;       // K2: waves per workgroup, one gate/up row pair each
static_assert(kGuWaves >= kDecMaxTokens, "K2 routes one token per wave");

__device__ __forceinline__ float dot8(uint4 w, uint4 x, float acc) {
  acc = fmaf(bf_lo(w.x), bf_lo(x.x), acc);
  acc = fmaf(bf_hi(w.x), bf_hi(x.x), acc);
  acc = fmaf(bf_lo(w.y), bf_lo(x.y), acc);
  acc = fmaf(bf_hi(w.y), bf_hi(x.y), acc);
  acc = fmaf(bf_lo(w.z), bf_lo(x.z), acc);
  acc = fmaf(bf_hi(w.z), bf_hi(x.z), acc);
  acc = fmaf(bf_lo(w.w), bf_lo(x.w), acc);
  acc = fmaf(bf_hi(w.w), bf_hi(x.w), acc);
  return acc;
}

template <bool FP8>
__device__ __forceinline__ const void* wrow(const void* base, long long row, int K) {
  return FP8 ? static_cast<const void*>(static_cast<const uint8_t*>(base) + row * K)
             : static_cast<const void*>(static_cast<const uint16_t*>(base) + row * K);
}

// Raw (undecoded) weight fragment, so that the loads of a whole row are issued before the
// first conversion.
template <bool FP8>
struct WFrag {
  uint4 v;
};
template <bool FP8>
__device__ __forceinline__ WFrag<FP8> ldraw(const void* row, int elem) {
  WFrag<FP8> f;
  if (FP8) {
    uint2 q = ld8_stream(static_cast<const uint8_t*>(row) + elem);
    f.v = make_uint4(q.x, q.y, 0u, 0u);
  } else {
    f.v = ld16_stream(static_cast<const uint16_t*>(row) + elem);
  }
  return f;
}
template <bool FP8>
__device__ __forceinline__ uint4 decode(WFrag<FP8> f) {
  if (FP8)
    return make_uint4(fp8x2_to_bf16x2<false>(f.v.x), fp8x2_to_bf16x2<true>(f.v.x),
                      fp8x2_to_bf16x2<false>(f.v.y), fp8x2_to_bf16x2<true>(f.v.y));
  return f.v;
}

__device__ __forceinline__ float swiglu(float g, float u) {
  return rbf(rbf(siluf_(rbf(g))) * rbf(u));
}

}  // namespace

// ------------------------------------------------------------------------------- K1

// grid: n_pack + IS (shared rows, when sh_gate) workgroups of one wave. The weight rows are
// requested before the token rows so that both are in flight together. With norm_x every
// wave normalises the token rows in registers (while its weight rows are in flight) and
// workgroup 0 stores them.
template <int NT, int HC>
__global__ __launch_bounds__(64) void k_dec_router(DecodeArgs a) {
  const int lane = threadIdx.x;
  const int g = blockIdx.x;
  const int H = HC * 512;
  const bool router = g < a.n_pack;
  const int n = g - a.n_pack;  // shared gate/up row pair
  const uint16_t* r0 = router ? a.w_pack + (long long)g * H : a.sh_gate + (long long)n * H;
  const uint16_t* r1 = router ? r0 : a.sh_up + (long long)n * H;
  uint4 w0[HC], w1[HC];
  uint4 xv[NT][HC];
  if (a.norm_x) {
    // post-attention add + RMSNorm of each token row, as k_add_rms computes it: the token
    // rows are requested first, then the weight rows, so the norm's arithmetic runs while
    // the weight rows are in flight
    uint4 tot[NT][HC], hv[NT][HC], wv[HC];
    const bool has_h = a.norm_h != nullptr;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const long long tr = (long long)min(t, a.T - 1) * H;
      load_row<HC, true>(a.norm_x + tr, H, lane, tot[t]);
      if (has_h) load_row<HC, true>(a.norm_h + tr, H, lane, hv[t]);
    }
    load_row<HC, true>(a.norm_w, H, lane, wv);
#pragma unroll
    for (int c = 0; c < HC; ++c) w0[c] = ld16_stream(r0 + c * 512 + lane * 8);
    if (!router) {
#pragma unroll
      for (int c = 0; c < HC; ++c) w1[c] = ld16_stream(r1 + c * 512 + lane * 8);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      add_rms_compute<HC>(has_h, H, a.norm_eps, tot[t], hv[t], wv, xv[t]);
      if (g == 0 && t < a.T) {
        const long long tr = (long long)t * H;
        if (has_h) store_row<HC>(a.norm_sum + tr, H, lane, tot[t]);
        store_row<HC>(a.norm_out + tr, H, lane, xv[t]);
      }
    }
  } else {
#pragma unroll
    for (int c = 0; c < HC; ++c) w0[c] = ld16_stream(r0 + c * 512 + lane * 8);
    if (!router) {
#pragma unroll
      for (int c = 0; c < HC; ++c) w1[c] = ld16_stream(r1 + c * 512 + lane * 8);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int c = 0; c < HC; ++c)
        xv[t][c] = ld16(a.x + (long long)min(t, a.T - 1) * H + c * 512 + lane * 8);
  }
  if (router) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      float s = 0.f;
#pragma unroll
      for (int c = 0; c < HC; ++c) s = dot8(w0[c], xv[t][c], s);
      s = wave_sum(s);
      if (lane == 0 && t < a.T) a.logits[(long long)t * a.n_pack + g] = f2bf_bits(s);
    }
    return;
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    float sg = 0.f, su = 0.f;
#pragma unroll
    for (int c = 0; c < HC; ++c) {
      sg = dot8(w0[c], xv[t][c], sg);
      su = dot8(w1[c], xv[t][c], su);
    }
    sg = wave_sum(sg);
    su = wave_sum(su);
    if (lane == 0 && t < a.T) a.act_sh[(long long)t * a.IS + n] = f2bf_bits(swiglu(sg, su));
  }
}

// ------------------------------------------------------------------------------- K2

// grid: [IS / kGuWaves shared row blocks when sh_in_gate_up] + P slots x (I / kGuWaves) row
// blocks; slots past the number of distinct experts exit. The shared expert's workgroups
// need no routing: their weight rows stream while the routed workgroups are still routing.
template <int NT, int HC, bool FP8, int EPL>
__global__ __launch_bounds__(64 * kGuWaves) void k_dec_gate_up(DecodeArgs a) {
  __shared__ int s_idx[64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int H = HC * 512;
  const int P = a.T * a.k;
  const int nrb = a.I / kGuWaves;
  const int nsh = a.sh_in_gate_up && a.sh_gate ? a.IS / kGuWaves : 0;

  // token rows: independent of the routing, requested first
  uint4 xv[NT][HC];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int c = 0; c < HC; ++c)
      xv[t][c] = ld16(a.x + (long long)min(t, a.T - 1) * H + c * 512 + lane * 8);

  if ((int)blockIdx.x < nsh) {
    // shared gate/up row pair n: the same dot products, in the same order, as in k_dec_router
    const int n = blockIdx.x * kGuWaves + wave;
    const uint16_t* rg = a.sh_gate + (long long)n * H;
    const uint16_t* ru = a.sh_up + (long long)n * H;
    uint4 wg[HC], wu[HC];
#pragma unroll
    for (int c = 0; c < HC; ++c) wg[c] = ld16_stream(rg + c * 512 + lane * 8);
#pragma unroll
    for (int c = 0; c < HC; ++c) wu[c] = ld16_stream(ru + c * 512 + lane * 8);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      float sg = 0.f, su = 0.f;
#pragma unroll
      for (int c = 0; c < HC; ++c) {
        sg = dot8(wg[c], xv[t][c], sg);
        su = dot8(wu[c], xv[t][c], su);
      }
      sg = wave_sum(sg);
      su = wave_sum(su);
      if (lane == 0 && t < a.T) a.act_sh[(long long)t * a.IS + n] = f2bf_bits(swiglu(sg, su));
    }
    return;
  }
  const int bid = blockIdx.x - nsh;
  const int slot = bid / nrb;
  const int n = (bid - slot * nrb) * kGuWaves + wave;

  WFrag<FP8> fg[HC], fu[HC];
  float scg = 1.f, scu = 1.f;  // fp8 row scales, requested with the rows
  // this workgroup's gate and up rows n of expert ex (and their scales), requested
  auto request = [&](int ex) {
    const long long b = (long long)ex * 2 * a.I;
    if (a.gu_scale) {
      scg = a.gu_scale[b + n];
      scu = a.gu_scale[b + a.I + n];
    }
    const void* rg = wrow<FP8>(a.gate_up, b + n, H);
    const void* ru = wrow<FP8>(a.gate_up, b + a.I + n, H);
#pragma unroll
    for (int c = 0; c < HC; ++c) {
      fg[c] = ldraw<FP8>(rg, c * 512 + lane * 8);
      fu[c] = ldraw<FP8>(ru, c * 512 + lane * 8);
    }
  };
  int e;                       // this workgroup's expert
  unsigned long long pmask;    // the pairs routed to it
  if (NT == 1 && a.logits) {
    // One token: its k experts are distinct and slot s takes the s-th selected one, so the
    // weight rows are requested as soon as selection round s has found it; the remaining
    // rounds, the softmax and the exactness check run while they are in flight. Where the
    // exact selection (rows whose p order differs from the logit order) gives another
    // expert for the slot, the rows are requested again.
    uint16_t raw[EPL];
    uint32_t keys[EPL];
    route_keys<EPL>(a.logits, a.E, lane, raw, keys);
    const int rounds = min(a.k + 1, a.E);
    uint32_t m = wave_max_u32(keys[0]);
    const uint32_t top = m;
    uint32_t sel = lane == 0 ? m : 0u;
    for (int j = 1; j <= slot; ++j) {
      m = route_next<EPL>(keys, m);
      sel = lane == j ? m : sel;
    }
    e = 0xffff - (int)(m & 0xffffu);
    request(e);
    for (int j = slot + 1; j < rounds; ++j) {
      m = route_next<EPL>(keys, m);
      sel = lane == j ? m : sel;
    }
    int my_idx;
    float my_w;
    route_finish<EPL>(raw, top, sel, rounds, a.E, a.k, lane, my_idx, my_w);
    const int e_exact = __builtin_amdgcn_readlane(my_idx, slot);
    if (e_exact != e) {
      e = e_exact;
      request(e);
    }
    pmask = __ballot(lane < a.k && my_idx == e);
    if (bid == 0 && wave == 0 && lane < a.k) {
      a.idx32[lane] = my_idx;
      a.wts[lane] = f2bf_bits(my_w);
      if (a.idx64) a.idx64[lane] = my_idx;
    }
  } else {
    // key: the expert of pair `lane` (lanes < P)
    if (a.logits) {
      if (wave < a.T) {
        int my_idx;
        float my_w;
        route_row<EPL>(a.logits + (long long)wave * a.n_pack, a.E, a.k, lane, my_idx, my_w);
        if (lane < a.k) {
          const int p = wave * a.k + lane;
          s_idx[p] = my_idx;
          if (bid == 0) {
            a.idx32[p] = my_idx;
            a.wts[p] = f2bf_bits(my_w);
            if (a.idx64) a.idx64[p] = my_idx;
          }
        }
      }
    } else if (threadIdx.x < P) {
      const long long v = a.ids_in[threadIdx.x];
      const int ev = (int)(v < 0 ? 0 : (v >= a.E ? a.E - 1 : v));
      s_idx[threadIdx.x] = ev;
      if (bid == 0) a.idx32[threadIdx.x] = ev;
    }
    __syncthreads();
    const int key = lane < P ? s_idx[lane] : -1;
    // distinct experts numbered in first-use order (pair order)
    bool first = lane < P;
    for (int q = 0; q < P; ++q) {
      const int kq = __builtin_amdgcn_readlane(key, q);
      if (q < lane && kq == key) first = false;
    }
    const unsigned long long fmask = __ballot(first);
    const int rank = __popcll(fmask & ((1ull << lane) - 1ull));
    if (slot >= __popcll(fmask)) return;
    const unsigned long long smask = __ballot(first && rank == slot);
    e = __builtin_amdgcn_readlane(key, __ffsll((long long)smask) - 1);
    pmask = __ballot(lane < P && key == e);
    request(e);
  }
  const long long base = (long long)e * 2 * a.I;
  float sg[NT], su[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) sg[t] = su[t] = 0.f;
#pragma unroll
  for (int c = 0; c < HC; ++c) {
    const uint4 wg = decode<FP8>(fg[c]);
    const uint4 wu = decode<FP8>(fu[c]);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      sg[t] = dot8(wg, xv[t][c], sg[t]);
      su[t] = dot8(wu, xv[t][c], su[t]);
    }
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    sg[t] = wave_sum(sg[t]) * scg;
    su[t] = wave_sum(su[t]) * scu;
  }
  // lane 0 writes each pair of this expert (at most one per token)
  while (pmask) {
    const int p = __ffsll((long long)pmask) - 1;
    pmask &= pmask - 1;
    const int t = p / a.k;
    float g = sg[0], u = su[0];
#pragma unroll
    for (int tt = 1; tt < NT; ++tt)
      if (t == tt) {
        g = sg[tt];
        u = su[tt];
      }
    if (lane == 0) a.act[(long long)p * a.I + n] = f2bf_bits(swiglu(g, u));
  }
}

// K2 for three or four tokens: each routed workgroup routes once and then takes G
// consecutive blocks of kGuWaves gate/up row pairs of its expert, requesting the rows of
// block g + 1 before multiplying block g (one routing and one round of workgroups instead
// of G: at four tokens the one-block kernel needs 5.5 rounds of resident workgroups, each
// paying the routing before its first weight request). The token rows are staged in LDS
// once per workgroup (read by its four waves and all G blocks) instead of being loaded by
// every wave: at four tokens the per-wave copies were twice the bytes of the weight rows
// and held 64 registers through the routing. Same dot products in the same order as
// k_dec_gate_up. grid: [IS / kGuWaves shared row blocks] + P slots x (I / kGuWaves / G)
// row-block groups.
template <int NT, int HC, bool FP8, int EPL, int G>
__global__ __launch_bounds__(64 * kGuWaves)
__attribute__((amdgpu_waves_per_eu(HC <= 4 ? 4 : 1))) void k_dec_gate_up_multi(DecodeArgs a) {
  static_assert(NT > 1 && NT <= kGuWaves, "one token routed per wave");
  constexpr int kRowU4 = HC * 64;        // 16-byte units of one token row
  __shared__ int s_idx[64];
  __shared__ uint4 s_x[NT * kRowU4];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int H = HC * 512;
  const int P = a.T * a.k;
  const int ngrp = a.I / kGuWaves / G;   // routed workgroups per slot
  const int nsh = a.sh_in_gate_up && a.sh_gate ? a.IS / kGuWaves : 0;

  if ((int)blockIdx.x < nsh) {
    // shared gate/up row pair n: no routing dependency (as in k_dec_gate_up)
    uint4 xv[NT][HC];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int c = 0; c < HC; ++c)
        xv[t][c] = ld16(a.x + (long long)min(t, a.T - 1) * H + c * 512 + lane * 8);
    const int n = blockIdx.x * kGuWaves + wave;
    const uint16_t* rg = a.sh_gate + (long long)n * H;
    const uint16_t* ru = a.sh_up + (long long)n * H;
    uint4 wg[HC], wu[HC];
#pragma unroll
    for (int c = 0; c < HC; ++c) wg[c] = ld16_stream(rg + c * 512 + lane * 8);
#pragma unroll
    for (int c = 0; c < HC; ++c) wu[c] = ld16_stream(ru + c * 512 + lane * 8);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      float sg = 0.f, su = 0.f;
#pragma unroll
      for (int c = 0; c < HC; ++c) {
        sg = dot8(wg[c], xv[t][c], sg);
        su = dot8(wu[c], xv[t][c], su);
      }
      sg = wave_sum(sg);
      su = wave_sum(su);
      if (lane == 0 && t < a.T) a.act_sh[(long long)t * a.IS + n] = f2bf_bits(swiglu(sg, su));
    }
    return;
  }
  const int bid = blockIdx.x - nsh;
  const int slot = bid / ngrp;
  const int blk0 = (bid - slot * ngrp) * G;  // first row block of this workgroup

  // token rows straight into LDS by DMA (no registers: the loads stay in flight through the
  // routing below and are waited for at the barrier after it)
  constexpr int kXUnits = NT * kRowU4;
  static_assert(kXUnits % (64 * kGuWaves) == 0, "whole waves of 16-byte units");
#pragma unroll
  for (int i = 0; i < kXUnits / (64 * kGuWaves); ++i) {
    const int u = threadIdx.x + i * 64 * kGuWaves;
    const int t = u / kRowU4;
    dma16(reinterpret_cast<const uint4*>(a.x + (long long)min(t, a.T - 1) * H) + (u - t * kRowU4),
          &s_x[i * 64 * kGuWaves + wave * 64]);
  }

  // routing: wave t routes token t; key of lane p = the expert of pair p (lanes < P)
  if (a.logits) {
    if (wave < a.T) {
      int my_idx;
      float my_w;
      route_row<EPL>(a.logits + (long long)wave * a.n_pack, a.E, a.k, lane, my_idx, my_w);
      if (lane < a.k) {
        const int p = wave * a.k + lane;
        s_idx[p] = my_idx;
        if (bid == 0) {
          a.idx32[p] = my_idx;
          a.wts[p] = f2bf_bits(my_w);
          if (a.idx64) a.idx64[p] = my_idx;
        }
      }
    }
  } else if (threadIdx.x < P) {
    const long long v = a.ids_in[threadIdx.x];
    const int ev = (int)(v < 0 ? 0 : (v >= a.E ? a.E - 1 : v));
    s_idx[threadIdx.x] = ev;
    if (bid == 0) a.idx32[threadIdx.x] = ev;
  }
  __builtin_amdgcn_s_waitcnt(0);  // this wave's token-row DMA loads have landed
  __syncthreads();
  const int key = lane < P ? s_idx[lane] : -1;
  // distinct experts numbered in first-use order (pair order)
  bool first = lane < P;
  for (int q = 0; q < P; ++q) {
    const int kq = __builtin_amdgcn_readlane(key, q);
    if (q < lane && kq == key) first = false;
  }
  const unsigned long long fmask = __ballot(first);
  const int rank = __popcll(fmask & ((1ull << lane) - 1ull));
  if (slot >= __popcll(fmask)) return;
  const unsigned long long smask = __ballot(first && rank == slot);
  const int e = __builtin_amdgcn_readlane(key, __ffsll((long long)smask) - 1);
  const unsigned long long pmask0 = __ballot(lane < P && key == e);
  const long long base = (long long)e * 2 * a.I;

  WFrag<FP8> fg[2][HC], fu[2][HC];
  float scg[2] = {1.f, 1.f}, scu[2] = {1.f, 1.f};
  auto request = [&](int buf, int n) __attribute__((always_inline)) {
    if (a.gu_scale) {
      scg[buf] = a.gu_scale[base + n];
      scu[buf] = a.gu_scale[base + a.I + n];
    }
    const void* rg = wrow<FP8>(a.gate_up, base + n, H);
    const void* ru = wrow<FP8>(a.gate_up, base + a.I + n, H);
#pragma unroll
    for (int c = 0; c < HC; ++c) {
      fg[buf][c] = ldraw<FP8>(rg, c * 512 + lane * 8);
      fu[buf][c] = ldraw<FP8>(ru, c * 512 + lane * 8);
    }
  };
  request(0, blk0 * kGuWaves + wave);
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int b = g & 1;
    const int n = (blk0 + g) * kGuWaves + wave;
    if (g + 1 < G) request(b ^ 1, (blk0 + g + 1) * kGuWaves + wave);
    float sg[NT], su[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) sg[t] = su[t] = 0.f;
#pragma unroll
    for (int c = 0; c < HC; ++c) {
      const uint4 wg = decode<FP8>(fg[b][c]);
      const uint4 wu = decode<FP8>(fu[b][c]);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const uint4 xv = s_x[t * kRowU4 + c * 64 + lane];
        sg[t] = dot8(wg, xv, sg[t]);
        su[t] = dot8(wu, xv, su[t]);
      }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      sg[t] = wave_sum(sg[t]) * scg[b];
      su[t] = wave_sum(su[t]) * scu[b];
    }
    // lane 0 writes each pair of this expert (at most one per token)
    unsigned long long pmask = pmask0;
    while (pmask) {
      const int p = __ffsll((long long)pmask) - 1;
      pmask &= pmask - 1;
      const int t = p / a.k;
      float gg = sg[0], uu = su[0];
#pragma unroll
      for (int tt = 1; tt < NT; ++tt)
        if (t == tt) {
          gg = sg[tt];
          uu = su[tt];
        }
      if (lane == 0) a.act[(long long)p * a.I + n] = f2bf_bits(swiglu(gg, uu));
    }
  }
}

// ------------------------------------------------------------------------------- K3

// grid: H / 4 workgroups; wave w computes hidden row 4 * blockIdx.x + w of every token.
template <int NT, int IC, bool FP8>
__global__ __launch_bounds__(kDecThreads) void k_dec_down(DecodeArgs a) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int I = IC * 512;
  const int P = a.T * a.k;
  const int H = a.H;
  const bool shared = a.sh_down != nullptr;
  const int isc = a.IS / 512;

  // shared row and the shared activations do not depend on the routing: request them first
  uint4 ws[2], xs[NT][2];
  if (shared) {
#pragma unroll
    for (int c = 0; c < 2; ++c)
      if (c < isc) ws[c] = ld16_stream(a.sh_down + (long long)n * a.IS + c * 512 + lane * 8);
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int c = 0; c < 2; ++c)
        if (c < isc)
          xs[t][c] = ld16(a.act_sh + (long long)min(t, a.T - 1) * a.IS + c * 512 + lane * 8);
  }
  // routing, shared-gate logit and residual of every token: one round trip together
  const int kv = lane < P ? a.idx32[lane] : 0;
  const float wv = lane < P ? bf_bits2f(a.wts[lane]) : 0.f;
  const int tl = min(lane, a.T - 1);
  // unconditional loads from always-valid addresses (a predicated load would be waited on
  // before the branch around it)
  const uint16_t* segp = shared ? a.logits + (long long)tl * a.n_pack + a.E : a.wts;
  const uint16_t* resp = a.residual ? a.residual + (long long)tl * H + n : a.wts;
  const float seg_l = bf_bits2f(*segp);
  const float res_l = bf_bits2f(*resp);

  float acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = 0.f;
  // pairs in groups of 8: all loads of a group are in flight before the first dot
  for (int p0 = 0; p0 < P; p0 += 8) {
    WFrag<FP8> wf[8][IC];
    uint4 av[8][IC];
    int ev[8];
    float dsc[8];  // fp8 row scales, requested with the rows
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int p = min(p0 + i, P - 1);
      ev[i] = __builtin_amdgcn_readlane(kv, p);
      dsc[i] = a.dn_scale ? a.dn_scale[(long long)ev[i] * H + n] : 1.f;
      const void* row = wrow<FP8>(a.down, (long long)ev[i] * H + n, I);
#pragma unroll
      for (int c = 0; c < IC; ++c) {
        wf[i][c] = ldraw<FP8>(row, c * 512 + lane * 8);
        av[i][c] = ld16(a.act + (long long)p * I + c * 512 + lane * 8);
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int p = p0 + i;
      if (p >= P) break;
      float s = 0.f;
#pragma unroll
      for (int c = 0; c < IC; ++c) s = dot8(decode<FP8>(wf[i][c]), av[i][c], s);
      s = wave_sum(s);
      s *= dsc[i];
      const float y = rbf(s);
      const float w = __shfl(wv, p);
      const float term = a.round_w ? rbf(w * y) : w * y;
      const int t = p / a.k;  // pairs run token-major, j ascending inside a token
#pragma unroll
      for (int tt = 0; tt < NT; ++tt)
        if (t == tt) acc[tt] += term;
    }
  }

  float o[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) o[t] = rbf(acc[t]);
  if (shared) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      float s = 0.f;
#pragma unroll
      for (int c = 0; c < 2; ++c)
        if (c < isc) s = dot8(ws[c], xs[t][c], s);
      s = wave_sum(s);
      const float gte = rbf(sigmoidf_(__shfl(seg_l, t)));
      o[t] = rbf(o[t] + rbf(gte * rbf(s)));
    }
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    if (t >= a.T) break;
    // lane t holds token t's residual
    if (lane == t) a.out[(long long)t * H + n] = f2bf_bits(a.residual ? o[t] + res_l : o[t]);
  }
}

// One token (T = 1, k <= 15): wave j < k owns pair j and wave k the shared expert; each
// wave streams kDownRows consecutive rows of its expert's down projection (contiguous
// memory) against its one activation row, and the combine runs over the waves' results in
// LDS in routing order. grid: H / kDownRows workgroups of (k + 1) waves.
constexpr int kDownRows = 4;  // measured at C2: 18.3 µs per layer against 18.8 (8 rows) and 18.4 (2)
template <int IC, bool FP8>
__global__ __launch_bounds__(1024) void k_dec_down1(DecodeArgs a) {
  __shared__ float s_term[16][kDownRows];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * kDownRows;
  const int I = IC * 512;
  const int H = a.H;
  const bool is_shared = wave == a.k;
  // the combine's other inputs (shared-expert gate logit, residual) requested up front, so
  // that no load waits after the barrier
  float seg_in = 0.f, res_in = 0.f;
  if (wave == 0 && lane < kDownRows) {
    if (a.sh_down) seg_in = bf_bits2f(a.logits[a.E]);
    if (a.residual) res_in = bf_bits2f(a.residual[n0 + lane]);
  }
  if (is_shared && a.sh_down) {
    // the shared expert: no routing dependency
    uint4 xs[2], ws[kDownRows][2];
    const int isc = a.IS / 512;
#pragma unroll
    for (int c = 0; c < 2; ++c)
      if (c < isc) {
#pragma unroll
        for (int r = 0; r < kDownRows; ++r)
          ws[r][c] = ld16_stream(a.sh_down + (long long)(n0 + r) * a.IS + c * 512 + lane * 8);
        xs[c] = ld16(a.act_sh + c * 512 + lane * 8);
      }
#pragma unroll
    for (int r = 0; r < kDownRows; ++r) {
      float d = 0.f;
#pragma unroll
      for (int c = 0; c < 2; ++c)
        if (c < isc) d = dot8(ws[r][c], xs[c], d);
      d = wave_sum(d);
      if (lane == r) s_term[15][r] = rbf(d);
    }
  } else if (!is_shared) {
    const int e = a.idx32[wave];
    const float w = bf_bits2f(a.wts[wave]);
    WFrag<FP8> wf[kDownRows][IC];
    uint4 av[IC];
#pragma unroll
    for (int c = 0; c < IC; ++c) av[c] = ld16(a.act + (long long)wave * I + c * 512 + lane * 8);
#pragma unroll
    for (int r = 0; r < kDownRows; ++r) {
      const void* row = wrow<FP8>(a.down, (long long)e * H + n0 + r, I);
#pragma unroll
      for (int c = 0; c < IC; ++c) wf[r][c] = ldraw<FP8>(row, c * 512 + lane * 8);
    }
    // fp8 row scales requested with the rows, not after the dot products
    float scl[kDownRows];
#pragma unroll
    for (int r = 0; r < kDownRows; ++r)
      scl[r] = a.dn_scale ? a.dn_scale[(long long)e * H + n0 + r] : 1.f;
#pragma unroll
    for (int r = 0; r < kDownRows; ++r) {
      float d = 0.f;
#pragma unroll
      for (int c = 0; c < IC; ++c) d = dot8(decode<FP8>(wf[r][c]), av[c], d);
      d = wave_sum(d);
      const float y = rbf(d * scl[r]);
      if (lane == r) s_term[wave][r] = a.round_w ? rbf(w * y) : w * y;
    }
  }
  __syncthreads();
  if (wave == 0 && lane < kDownRows) {
    const int n = n0 + lane;
    float acc = 0.f;
    for (int j = 0; j < a.k; ++j) acc += s_term[j][lane];  // routing order j
    float o = rbf(acc);
    if (a.sh_down) {
      const float gte = rbf(sigmoidf_(seg_in));
      o = rbf(o + rbf(gte * s_term[15][lane]));
    }
    if (a.residual) o += res_in;
    a.out[n] = f2bf_bits(o);
  }
}

// ------------------------------------------------------------------------ host side

bool decode_fits(const DecodeArgs& a) {
  const int P = a.T * a.k;
  if (a.T < 1 || a.T > kDecMaxTokens || P > 64 || a.k < 1) return false;
  // hidden sizes of the instantiated kernels: 512 times 1, 2, 4 or 8
  const int hc = a.H / 512;
  if (a.H % 512 || (hc != 1 && hc != 2 && hc != 4 && hc != 8)) return false;
  if (a.I % 512 || a.I > 1024 || a.I < 512) return false;
  if (a.logits && (a.E > 512 || a.E < 1)) return false;
  if (a.sh_down && (a.IS % 512 || a.IS > 1024 || a.IS < 512)) return false;
  return true;
}

namespace {

// Row blocks per routed K2 workgroup at three or four tokens: MOE_DECODE_GU_BLOCKS=1, 2
// or 4 (comparisons; 1 is the one-block kernel that loads the token rows per wave).
int gate_up_blocks() {
  const char* env = knob(kKnobDecodeGuBlocks);
  const int v = env ? atoi(env) : 4;
  return v == 1 || v == 2 ? v : 4;
}

// MOE_DECODE_DOWN=rows: the wave-per-row down kernel for one token too (comparisons).
bool down_legacy() {
  const char* env = knob(kKnobDecodeDown);
  return env && env[0] == 'r';
}

template <int NT>
hipError_t launch_router_nt(const DecodeArgs& a, hipStream_t s) {
  const int grid = a.n_pack + (a.sh_gate && !a.sh_in_gate_up ? a.IS : 0);
  switch (a.H / 512) {
#define L(HC)                                                                             \
  case HC:                                                                                \
    hipLaunchKernelGGL((k_dec_router<NT, HC>), dim3(grid), dim3(64), 0, s, a); \
    break;
    L(1) L(2) L(4) L(8)
#undef L
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int NT, bool FP8>
hipError_t launch_gate_up_nt(const DecodeArgs& a, hipStream_t s) {
  // three or four tokens: G row blocks per routed workgroup (I / kGuWaves is a multiple of 4)
  const int G = NT == 4 ? gate_up_blocks() : 1;
  const bool multi = G > 1;
  const int grid = a.T * a.k * (a.I / kGuWaves / G) +
                   (a.sh_gate && a.sh_in_gate_up ? a.IS / kGuWaves : 0);
  const int epl = a.logits ? (a.E + 63) / 64 : 1;
#define LG(HC, EPL)                                                                         \
  if (a.H / 512 == HC && epl <= EPL) {                                                      \
    if (multi && G == 4)                                                                    \
      hipLaunchKernelGGL((k_dec_gate_up_multi<4, HC, FP8, EPL, 4>), dim3(grid),             \
                         dim3(64 * kGuWaves), 0, s, a);                                     \
    else if (multi)                                                                         \
      hipLaunchKernelGGL((k_dec_gate_up_multi<4, HC, FP8, EPL, 2>), dim3(grid),             \
                         dim3(64 * kGuWaves), 0, s, a);                                     \
    else                                                                                    \
      hipLaunchKernelGGL((k_dec_gate_up<NT, HC, FP8, EPL>), dim3(grid), dim3(64 * kGuWaves), 0, s, a); \
    return hipGetLastError();                                                               \
  }
#define LH(HC) LG(HC, 1) LG(HC, 2) LG(HC, 4) LG(HC, 8)
  LH(1) LH(2) LH(4) LH(8)
#undef LH
#undef LG
  return hipErrorInvalidValue;
}

template <int NT, bool FP8>
hipError_t launch_down_nt(const DecodeArgs& a, hipStream_t s) {
  if (NT == 1 && a.T == 1 && a.k <= 15 && a.H % kDownRows == 0 && !down_legacy()) {
    const int grid = a.H / kDownRows;
    const dim3 block(64 * (a.k + 1));
    if (a.I == 512)
      hipLaunchKernelGGL((k_dec_down1<1, FP8>), dim3(grid), block, 0, s, a);
    else if (a.I == 1024)
      hipLaunchKernelGGL((k_dec_down1<2, FP8>), dim3(grid), block, 0, s, a);
    else
      return hipErrorInvalidValue;
    return hipGetLastError();
  }
  const int grid = a.H / 4;
  if (a.I == 512)
    hipLaunchKernelGGL((k_dec_down<NT, 1, FP8>), dim3(grid), dim3(kDecThreads), 0, s, a);
  else if (a.I == 1024)
    hipLaunchKernelGGL((k_dec_down<NT, 2, FP8>), dim3(grid), dim3(kDecThreads), 0, s, a);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace

hipError_t launch_decode_router(const DecodeArgs& a, hipStream_t s) {
  if (a.T == 1) return launch_router_nt<1>(a, s);
  if (a.T == 2) return launch_router_nt<2>(a, s);
  return launch_router_nt<4>(a, s);
}

hipError_t launch_decode_gate_up(const DecodeArgs& a, hipStream_t s) {
  if (a.fp8) {
    if (a.T == 1) return launch_gate_up_nt<1, true>(a, s);
    if (a.T == 2) return launch_gate_up_nt<2, true>(a, s);
    return launch_gate_up_nt<4, true>(a, s);
  }
  if (a.T == 1) return launch_gate_up_nt<1, false>(a, s);
  if (a.T == 2) return launch_gate_up_nt<2, false>(a, s);
  return launch_gate_up_nt<4, false>(a, s);
}

hipError_t launch_decode_down(const DecodeArgs& a, hipStream_t s) {
  if (a.fp8) {
    if (a.T == 1) return launch_down_nt<1, true>(a, s);
    if (a.T == 2) return launch_down_nt<2, true>(a, s);
    return launch_down_nt<4, true>(a, s);
  }
  if (a.T == 1) return launch_down_nt<1, false>(a, s);
  if (a.T == 2) return launch_down_nt<2, false>(a, s);
  return launch_down_nt<4, false>(a, s);
}

}  // namespace moe
