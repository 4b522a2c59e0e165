// Device-side routing (softmax / top-k) and sort helpers shared by the standalone
// route / sort kernels (route_sort.hip) and the router GEMM's fused routing tail
// (expert_gemm.hip). See route_sort.hip for the contract.
#pragma once
#include "moe_common.h"

namespace moe {

constexpr int kSortThreads = 1024;
constexpr int kSortWaves = kSortThreads / kWave;
constexpr int kSmallMaxPairs = 4096;
constexpr int kSmallMaxE = 512;
constexpr int kMaxE = 1024;

// ---------------------------------------------------------------------------- routing

// Wave-wide reductions without LDS round trips: DPP within each 16-lane row (quad xor 1,
// quad xor 2, half-row mirror, row mirror leave the row's result in all 16 lanes), then
// the four rows combined from readlanes in a fixed order. Deterministic.
constexpr int kDppXor1 = 0xB1;        // quad_perm(1, 0, 3, 2)
constexpr int kDppXor2 = 0x4E;        // quad_perm(2, 3, 0, 1)
constexpr int kDppHalfMirror = 0x141;  // row_half_mirror
constexpr int kDppMirror = 0x140;      // row_mirror

template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dppi(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ float rowlane(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dppf<kDppXor1>(v));
  v = fmaxf(v, dppf<kDppXor2>(v));
  v = fmaxf(v, dppf<kDppHalfMirror>(v));
  v = fmaxf(v, dppf<kDppMirror>(v));
  return fmaxf(fmaxf(rowlane(v, 0), rowlane(v, 16)), fmaxf(rowlane(v, 32), rowlane(v, 48)));
}
__device__ __forceinline__ float wave_sum(float v) {
  v += dppf<kDppXor1>(v);
  v += dppf<kDppXor2>(v);
  v += dppf<kDppHalfMirror>(v);
  v += dppf<kDppMirror>(v);
  return (rowlane(v, 0) + rowlane(v, 16)) + (rowlane(v, 32) + rowlane(v, 48));
}

// (p, expert) pair order of the routing: larger p first, the lower expert on ties.
__device__ __forceinline__ bool better(float pa, int ia, float pb, int ib) {
  return pa > pb || (pa == pb && ia < ib);
}
template <int CTRL>
__device__ __forceinline__ void argmax_dpp(float& v, int& i) {
  float ov = dppf<CTRL>(v);
  int oi = dppi<CTRL>(i);
  if (better(ov, oi, v, i)) {
    v = ov;
    i = oi;
  }
}
// Wave-uniform argmax of (v, i) under ``better``.
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
  argmax_dpp<kDppXor1>(v, i);
  argmax_dpp<kDppXor2>(v, i);
  argmax_dpp<kDppHalfMirror>(v, i);
  argmax_dpp<kDppMirror>(v, i);
  float bv = rowlane(v, 0);
  int bi = __builtin_amdgcn_readlane(i, 0);
#pragma unroll
  for (int r = 16; r < 64; r += 16) {
    float ov = rowlane(v, r);
    int oi = __builtin_amdgcn_readlane(i, r);
    if (better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  v = bv;
  i = bi;
}

template <int EPL>
__device__ void route_row(const uint16_t* __restrict__ lrow, int E, int k, int lane,
                          int& my_idx, float& my_w) {
  float p[EPL];
  float m = -INFINITY;
  // all EPL loads in flight at once (clamped addresses, masked after): one memory round
  // trip, not one per element
  uint16_t raw[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) raw[i] = lrow[min(lane + kWave * i, E - 1)];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    int e = lane + kWave * i;
    float z = e < E ? bf_bits2f(raw[i]) : -INFINITY;
    p[i] = z;
    m = fmaxf(m, z);
  }
  m = wave_max(m);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    int e = lane + kWave * i;
    p[i] = e < E ? expf(p[i] - m) : 0.f;
    s += p[i];
  }
  s = wave_sum(s);
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    int e = lane + kWave * i;
    p[i] = e < E ? p[i] / s : -1.0f;
  }
  float tot = 0.f;
  float mine_p = 0.f;
  int mine_i = 0;
  for (int j = 0; j < k; ++j) {
    float bp = -2.0f;
    int bi = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < EPL; ++i)
      if (p[i] > bp) {  // strict: the lowest expert of the lane wins a tie
        bp = p[i];
        bi = lane + kWave * i;
      }
    wave_argmax(bp, bi);
#pragma unroll
    for (int i = 0; i < EPL; ++i)
      if (lane + kWave * i == bi) p[i] = -1.0f;
    tot += bp;  // sequential j order
    if (lane == j) {
      mine_p = bp;
      mine_i = bi;
    }
  }
  my_idx = mine_i;
  my_w = mine_p / tot;
}

template <int EPL>
__device__ void route_rows(const uint16_t* __restrict__ logits, long long ld, int t, int E, int k,
                           int lane, long long* __restrict__ idx64, int* __restrict__ idx32,
                           uint16_t* __restrict__ w_out, int* __restrict__ keys_lds,
                           int* __restrict__ counts_g) {
  int my_i;
  float my_w;
  route_row<EPL>(logits + (long long)t * ld, E, k, lane, my_i, my_w);
  if (lane < k) {
    long long pidx = (long long)t * k + lane;
    if (idx64) idx64[pidx] = my_i;
    if (idx32) idx32[pidx] = my_i;
    if (w_out) w_out[pidx] = f2bf_bits(my_w);
    if (keys_lds) keys_lds[pidx] = my_i;
    if (counts_g) atomicAdd(counts_g + my_i, 1);
  }
}

// ------------------------------------------------------------------ block-level helpers

// Exclusive scan of one int per thread over the whole block (<= 1024 threads).
__device__ int block_excl_scan(int v, int* tmp, int& total) {
  int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    int y = __shfl_up(x, off);
    if (lane >= off) x += y;
  }
  if (lane == 63) tmp[w] = x;
  __syncthreads();
  if (w == 0) {
    int t = lane < nw ? tmp[lane] : 0;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      int y = __shfl_up(t, off);
      if (lane >= off) t += y;
    }
    if (lane < nw) tmp[lane] = t;
  }
  __syncthreads();
  int base = w > 0 ? tmp[w - 1] : 0;
  total = tmp[nw - 1];
  __syncthreads();
  return base + x - v;
}

// From per-expert counts in LDS: global counts / offsets, the offsets in LDS, and the
// tile table. Requires E <= blockDim.x.
__device__ void build_table(const int* cnt, int E, int P, int T, int bm, int has_shared,
                            int* offs_lds, int* __restrict__ counts_g, int* __restrict__ offsets_g,
                            int* __restrict__ table, int MT, int* tmp) {
  int e = threadIdx.x;
  int c = e < E ? cnt[e] : 0;
  int total;
  int st = block_excl_scan(c, tmp, total);
  int nt = (c + bm - 1) / bm;
  int ntot;
  int tst = block_excl_scan(nt, tmp, ntot);
  if (e < E) {
    offs_lds[e] = st;
    if (counts_g) counts_g[e] = c;
    if (offsets_g) offsets_g[e] = st;
    for (int j = 0; j < nt; ++j) {
      int t = tst + j;
      table[t] = e;
      table[MT + t] = st + j * bm;
      table[2 * MT + t] = st + c;
    }
  }
  int nsh = has_shared ? (T + bm - 1) / bm : 0;
  for (int j = threadIdx.x; j < nsh; j += blockDim.x) {
    int t = ntot + j;
    table[t] = E;
    table[MT + t] = P + j * bm;
    table[2 * MT + t] = P + T;
  }
  if (threadIdx.x == 0) table[3 * MT] = ntot + nsh;
  __syncthreads();
}

// Stable in-block ranks: thread i holds key (valid when valid). Returns the number of
// valid keys equal to key at lower thread ids of the block. wcnt is [waves][E] in LDS.
__device__ int block_stable_rank(int key, bool valid, int E, int nbits, int* wcnt) {
  int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  for (int i = threadIdx.x; i < nw * E; i += blockDim.x) wcnt[i] = 0;
  __syncthreads();
  unsigned long long m = __ballot(valid);
  for (int b = 0; b < nbits; ++b) {
    bool bit = (key >> b) & 1;
    unsigned long long bb = __ballot(bit);
    m &= bit ? bb : ~bb;
  }
  int rank = __popcll(m & ((1ull << lane) - 1ull));
  if (valid && rank == 0) wcnt[w * E + key] = __popcll(m);
  __syncthreads();
  if (valid)
    for (int v = 0; v < w; ++v) rank += wcnt[v * E + key];
  return rank;
}

// LDS of the one-workgroup route + sort (blockDim.x <= 1024, E <= min(blockDim.x, 512)).
struct SortLds {
  int keys[kSmallMaxPairs];
  int hist[kSmallMaxE];
  int offs[kSmallMaxE];
  int wcnt[kSortWaves * kSmallMaxE];
  int tmp[kSortWaves + 1];
};

// One workgroup: (optionally) route T rows, then count, scan, build the tile table and
// scatter the stable order. P = T * k <= kSmallMaxPairs, E <= min(blockDim.x, kSmallMaxE).
template <int EPL>
__device__ void route_sort_block(const uint16_t* __restrict__ logits, long long ld,
                                 const int* __restrict__ ids32_in,
                                 const long long* __restrict__ ids64_in, int T, int E, int k,
                                 int bm, int has_shared, long long* __restrict__ idx64,
                                 int* __restrict__ idx32, uint16_t* __restrict__ w_out,
                                 int* __restrict__ counts_g, int* __restrict__ offsets_g,
                                 int* __restrict__ order, int* __restrict__ table, int MT,
                                 SortLds& L) {
  const int P = T * k;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  for (int e = threadIdx.x; e < E; e += blockDim.x) L.hist[e] = 0;
  if (logits) {
    for (int t = wave; t < T; t += nw)
      route_rows<EPL>(logits, ld, t, E, k, lane, idx64, idx32, w_out, L.keys, nullptr);
  } else {
    for (int p = threadIdx.x; p < P; p += blockDim.x) {
      long long v = ids64_in ? ids64_in[p] : (long long)ids32_in[p];
      L.keys[p] = (int)(v < 0 ? 0 : (v >= E ? E - 1 : v));  // clamp as batched_mm does
    }
  }
  __syncthreads();
  for (int p = threadIdx.x; p < P; p += blockDim.x) atomicAdd(&L.hist[L.keys[p]], 1);
  __syncthreads();
  build_table(L.hist, E, P, T, bm, has_shared, L.offs, counts_g, offsets_g, table, MT, L.tmp);
  const int nbits = E > 1 ? 32 - __clz(E - 1) : 1;
  for (int c0 = 0; c0 < P; c0 += blockDim.x) {
    int p = c0 + threadIdx.x;
    bool valid = p < P;
    int key = valid ? L.keys[p] : 0;
    int rank = block_stable_rank(key, valid, E, nbits, L.wcnt);
    if (valid) order[L.offs[key] + rank] = p;
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
      int s = 0;
      for (int v = 0; v < nw; ++v) s += L.wcnt[v * E + e];
      L.offs[e] += s;
    }
    __syncthreads();
  }
}

#define MOE_EPL_DISPATCH(E, FN)       \
  do {                                \
    if ((E) <= 64) {                  \
      FN(1);                          \
    } else if ((E) <= 128) {          \
      FN(2);                          \
    } else if ((E) <= 256) {          \
      FN(4);                          \
    } else if ((E) <= 512) {          \
      FN(8);                          \
    } else {                          \
      FN(16);                         \
    }                                 \
  } while (0)

}  // namespace moe
