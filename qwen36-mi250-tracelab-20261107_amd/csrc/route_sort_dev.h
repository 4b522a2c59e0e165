// Device-side routing (softmax / top-k) and sort helpers shared by the standalone
// route / sort kernels (route_sort.hip) and the decode gate_up kernel (decode.hip). See
// route_sort.hip for the contract.
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

constexpr int kDppBcast15 = 0x142;  // row_bcast:15 (rows 1, 3 <- last lane of the row before)
constexpr int kDppBcast31 = 0x143;  // row_bcast:31 (rows 2, 3 <- lane 31)

template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ uint32_t max_dpp_u32(uint32_t v) {
  // lanes outside ROWS (and invalid sources) read 0, the identity of the max
  const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWS, 0xF, true);
  return o > v ? o : v;
}
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ int min_dpp_i32(int v) {
  const int o = __builtin_amdgcn_update_dpp(0x7fffffff, v, CTRL, ROWS, 0xF, false);
  return o < v ? o : v;
}
// Wave-uniform max / min: DPP within rows, row broadcasts across them (lane 63 ends with
// the result), one readlane. No branches, no LDS.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max_dpp_u32<kDppXor1>(v);
  v = max_dpp_u32<kDppXor2>(v);
  v = max_dpp_u32<kDppHalfMirror>(v);
  v = max_dpp_u32<kDppMirror>(v);
  v = max_dpp_u32<kDppBcast15, 0xA>(v);
  v = max_dpp_u32<kDppBcast31, 0xC>(v);
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}
__device__ __forceinline__ int wave_min_i32(int v) {
  v = min_dpp_i32<kDppXor1>(v);
  v = min_dpp_i32<kDppXor2>(v);
  v = min_dpp_i32<kDppHalfMirror>(v);
  v = min_dpp_i32<kDppMirror>(v);
  v = min_dpp_i32<kDppBcast15, 0xA>(v);
  v = min_dpp_i32<kDppBcast31, 0xC>(v);
  return __builtin_amdgcn_readlane(v, 63);
}

// Routing order of (p, expert) entries: larger p first, the lower expert on equal p. p >= 0,
// so its fp32 bits order like its values; empty entries carry p bits 0 and expert INT_MAX
// (below every real entry: equal p bits resolve to the lower expert).
__device__ __forceinline__ bool route_before(uint32_t pa, int ea, uint32_t pb, int eb) {
  return pa > pb || (pa == pb && ea < eb);
}
__device__ __forceinline__ void cas_desc(uint32_t& pa, int& ea, uint32_t& pb, int& eb) {
  const bool sw = route_before(pb, eb, pa, ea);
  const uint32_t tp = pa;
  const int te = ea;
  pa = sw ? pb : pa;
  ea = sw ? eb : ea;
  pb = sw ? tp : pb;
  eb = sw ? te : eb;
}

// Exact selection on the probabilities: each lane's EPL entries sorted in routing order,
// k rounds take the wave maximum of the lanes' head p and pop the winning head; equal p in
// several lanes go to the lowest expert through a second reduction.
template <int EPL>
__device__ void route_select_exact(const float* p, int E, int k, int lane, float& mine_p,
                                   int& mine_i, float& tot) {
  uint32_t kp[EPL];
  int ke[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    int e = lane + kWave * i;
    kp[i] = e < E ? __float_as_uint(p[i]) : 0u;
    ke[i] = e < E ? e : 0x7fffffff;
  }
#pragma unroll
  for (int w = 1; w < EPL; ++w)  // insertion network
#pragma unroll
    for (int i = w; i > 0; --i) cas_desc(kp[i - 1], ke[i - 1], kp[i], ke[i]);
  tot = 0.f;
  for (int j = 0; j < k; ++j) {
    const uint32_t m = wave_max_u32(kp[0]);
    bool win = kp[0] == m;
    const unsigned long long bal = __ballot(win);
    int e_win;
    if (__popcll(bal) == 1) {
      e_win = __builtin_amdgcn_readlane(ke[0], __ffsll((long long)bal) - 1);
    } else {
      e_win = wave_min_i32(win ? ke[0] : 0x7fffffff);
      win = win && ke[0] == e_win;
    }
#pragma unroll
    for (int i = 0; i + 1 < EPL; ++i) {
      kp[i] = win ? kp[i + 1] : kp[i];
      ke[i] = win ? ke[i + 1] : ke[i];
    }
    if (win) {
      kp[EPL - 1] = 0u;
      ke[EPL - 1] = 0x7fffffff;
    }
    const float bp = __uint_as_float(m);
    tot += bp;  // sequential j order
    if (lane == j) {
      mine_p = bp;
      mine_i = e_win;
    }
  }
}

// bf16 logit -> 16-bit key that orders like the value (sign flipped, negatives inverted).
__device__ __forceinline__ uint32_t bf16_order_key(uint32_t b) {
  return (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
}
__device__ __forceinline__ uint32_t bf16_from_order_key(uint32_t k) {
  return (k & 0x8000u) ? (k & 0x7fffu) : (~k & 0xffffu);
}

// Softmax / top-k / renormalise of one token's E logits (one wave; lane j < k receives
// the j-th expert and its weight p_j / sum p_sel). Order: larger p first, the lower expert
// on equal p (the reference's rule on fp32 p = softmax(bf16 logits)).
//
// p is a non-decreasing function of the logit, so the k + 1 largest logits (ties to the
// lower expert: one 32-bit key per entry) are the k largest p in the same order whenever
// their p strictly decrease wherever their logits do. That is checked on the selection,
// and the cases that fail it (p equal for different logits, e.g. exp underflow; a boundary
// logit under 2^-10 in magnitude or a subnormal boundary p, where fp32 exp need not separate
// neighbouring logits) take the exact selection on p.
// Order keys of one row's logits (lane l holds entries l + 64 i, i < EPL), sorted
// descending per lane: key = (order key of the bf16 logit) << 16 | (0xffff - expert).
template <int EPL>
__device__ __forceinline__ void route_keys_raw(const uint16_t (&raw)[EPL], int E, int lane,
                                               uint32_t (&key)[EPL]) {
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    int e = lane + kWave * i;
    key[i] = e < E ? (bf16_order_key(raw[i]) << 16) | (uint32_t)(0xffff - e) : 0u;
  }
#pragma unroll
  for (int w = 1; w < EPL; ++w)  // insertion network, descending
#pragma unroll
    for (int i = w; i > 0; --i) {
      const uint32_t hi = max(key[i - 1], key[i]), lo = min(key[i - 1], key[i]);
      key[i - 1] = hi;
      key[i] = lo;
    }
}
template <int EPL>
__device__ __forceinline__ void route_keys(const uint16_t* __restrict__ lrow, int E, int lane,
                                           uint16_t (&raw)[EPL], uint32_t (&key)[EPL]) {
  // all EPL loads in flight at once (clamped addresses, masked after)
#pragma unroll
  for (int i = 0; i < EPL; ++i) raw[i] = lrow[min(lane + kWave * i, E - 1)];
  route_keys_raw<EPL>(raw, E, lane, key);
}

// One selection round: the previous round's winner (the lane whose head key is m; keys
// are distinct) drops its head key; returns the new wave maximum.
template <int EPL>
__device__ __forceinline__ uint32_t route_next(uint32_t (&key)[EPL], uint32_t m) {
  const bool win = key[0] == m;
#pragma unroll
  for (int i = 0; i + 1 < EPL; ++i) key[i] = win ? key[i + 1] : key[i];
  key[EPL - 1] = win ? 0u : key[EPL - 1];
  return wave_max_u32(key[0]);
}

// Softmax over the row and the selected entries' weights, from the first round's maximum
// (top) and the selected keys (lane j < rounds holds the j-th), with the exact-p fallback.
template <int EPL>
__device__ void route_finish(const uint16_t (&raw)[EPL], uint32_t top, uint32_t sel, int rounds,
                             int E, int k, int lane, int& my_idx, float& my_w) {
  const float mz = bf_bits2f(bf16_from_order_key(top >> 16));
  float p[EPL];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    int e = lane + kWave * i;
    p[i] = e < E ? expf(bf_bits2f(raw[i]) - mz) : 0.f;
    s += p[i];
  }
  s = wave_sum(s);
  // p of the selected entries, with the same operations as every other entry's
  const uint32_t zb = bf16_from_order_key(sel >> 16);
  const float ps = expf(bf_bits2f(zb) - mz) / s;
  const float pn = __shfl_down(ps, 1);
  const uint32_t kn = (uint32_t)__shfl_down((int)sel, 1);
  bool bad = false;
  if (lane + 1 < rounds) bad = !(ps > pn) && (sel >> 16) != (kn >> 16);
  // boundary entry: its logit at least 2^-10 in magnitude (distinct bf16 logits near it then
  // differ by >= 2^-18, >= 16 ulps of exp) and its p a normal number
  if (lane == k && lane < rounds) bad = !(fabsf(bf_bits2f(zb)) >= 0x1p-10f) || !(ps >= 0x1p-100f);
  float mine_p = 0.f, tot = 0.f;
  int mine_i = 0;
  if (__ballot(bad) == 0ull) {
    mine_p = ps;
    mine_i = 0xffff - (int)(sel & 0xffffu);
    for (int j = 0; j < k; ++j)  // sequential j order
      tot += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ps), j));
  } else {
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      int e = lane + kWave * i;
      p[i] = e < E ? p[i] / s : -1.0f;
    }
    route_select_exact<EPL>(p, E, k, lane, mine_p, mine_i, tot);
  }
  my_idx = mine_i;
  my_w = mine_p / tot;
}

// route_row on logits already in registers (lane l: entries l + 64 i; raw is read only for
// entries below E).
template <int EPL>
__device__ void route_row_raw(const uint16_t (&raw)[EPL], int E, int k, int lane, int& my_idx,
                              float& my_w) {
  uint32_t key[EPL];
  route_keys_raw<EPL>(raw, E, lane, key);
  const int rounds = min(k + 1, E);
  uint32_t m = wave_max_u32(key[0]);
  const uint32_t top = m;
  uint32_t sel = lane == 0 ? m : 0u;
  for (int j = 1; j < rounds; ++j) {
    m = route_next<EPL>(key, m);
    sel = lane == j ? m : sel;
  }
  route_finish<EPL>(raw, top, sel, rounds, E, k, lane, my_idx, my_w);
}

template <int EPL>
__device__ void route_row(const uint16_t* __restrict__ lrow, int E, int k, int lane,
                          int& my_idx, float& my_w) {
  uint16_t raw[EPL];
  uint32_t key[EPL];
  route_keys<EPL>(lrow, E, lane, raw, key);
  // k + 1 rounds: lane j keeps the j-th key (lane k: the first one not selected)
  const int rounds = min(k + 1, E);
  uint32_t m = wave_max_u32(key[0]);
  const uint32_t top = m;
  uint32_t sel = lane == 0 ? m : 0u;
  for (int j = 1; j < rounds; ++j) {
    m = route_next<EPL>(key, m);
    sel = lane == j ? m : sel;
  }
  route_finish<EPL>(raw, top, sel, rounds, E, k, lane, my_idx, my_w);
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

// Two rows of one wave (t1 < 0: none), their key set-up and selection rounds interleaved:
// the rounds are chains of dependent cross-lane steps, so two independent chains fill each
// other's wait slots. Each row's result is that of route_rows on it alone.
template <int EPL>
__device__ void route_rows2(const uint16_t* __restrict__ logits, long long ld, int t0, int t1,
                            int E, int k, int lane, long long* __restrict__ idx64,
                            int* __restrict__ idx32, uint16_t* __restrict__ w_out,
                            int* __restrict__ keys_lds, int* __restrict__ counts_g) {
  const int ts[2] = {t0, t1 < 0 ? t0 : t1};
  uint16_t raw[2][EPL];
  uint32_t key[2][EPL];
#pragma unroll
  for (int r = 0; r < 2; ++r) route_keys<EPL>(logits + (long long)ts[r] * ld, E, lane, raw[r], key[r]);
  const int rounds = min(k + 1, E);
  uint32_t m[2], top[2], sel[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    m[r] = wave_max_u32(key[r][0]);
    top[r] = m[r];
    sel[r] = lane == 0 ? m[r] : 0u;
  }
  for (int j = 1; j < rounds; ++j) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      m[r] = route_next<EPL>(key[r], m[r]);
      sel[r] = lane == j ? m[r] : sel[r];
    }
  }
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    if (r == 1 && t1 < 0) break;
    int my_i;
    float my_w;
    route_finish<EPL>(raw[r], top[r], sel[r], rounds, E, k, lane, my_i, my_w);
    if (lane < k) {
      const long long pidx = (long long)ts[r] * k + lane;
      if (idx64) idx64[pidx] = my_i;
      if (idx32) idx32[pidx] = my_i;
      if (w_out) w_out[pidx] = f2bf_bits(my_w);
      if (keys_lds) keys_lds[pidx] = my_i;
      if (counts_g) atomicAdd(counts_g + my_i, 1);
    }
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
    // two tokens per pass of a wave, interleaved
    for (int t = wave; t < T; t += 2 * nw)
      route_rows2<EPL>(logits, ld, t, t + nw < T ? t + nw : -1, E, k, lane, idx64, idx32, w_out,
                       L.keys, nullptr);
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
