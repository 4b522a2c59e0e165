// Router softmax / top-k (subsystem a2) and the expert count / stable sort /
// tile table (subsystem a3) for gfx950.
//
// Routing follows the reference kernels' rule (engine/fast/prefill_kernels.py:194-219,
// engine/fast/fused.py:553-570): p = softmax_fp32(bf16 logits); the k largest p in
// descending order, ties to the lower expert index; weights bf16(p_sel / sum p_sel).
//
// The sort is a stable counting sort of the flattened pair expert ids (pair
// p = token * k + j): order[r] is the pair at sorted row r, identical to
// torch.argsort(ids, stable=True) (engine/experts.py:71, engine/fast/moe_prefill.py:562).
// It is deterministic (the reference's atomic-cursor order, prefill_kernels.py:221-230,
// is not): ranks inside a wave come from ballot masks over the key bits, ranks
// across waves from per-wave counts in LDS.
//
// The tile table has the layout of engine/fast/moe_prefill.py:92-154 (expert, first
// row, row end per BM-row tile; the tile count at 3 * max_tiles), plus optional
// "shared expert" tiles appended after the routed ones: expert id E, rows P + j*BM
// up to P + T (the shared expert sees every token).
#include "moe_common.h"

namespace moe {

constexpr int kSortThreads = 1024;
constexpr int kSortWaves = kSortThreads / kWave;
constexpr int kSmallMaxPairs = 4096;
constexpr int kSmallMaxE = 512;
constexpr int kMaxE = 1024;

// ---------------------------------------------------------------------------- routing

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// One wave routes one row of E bf16 logits. Lane l owns experts l, l+64, ...
// Writes (for lanes j < k) sel_idx / sel_w of pick j through the callback arrays.
template <int EPL>
__device__ void route_row(const uint16_t* __restrict__ lrow, int E, int k, int lane,
                          int& my_idx, float& my_w) {
  float p[EPL];
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    int e = lane + kWave * i;
    float z = e < E ? bf_bits2f(lrow[e]) : -INFINITY;
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
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      float op = __shfl_xor(bp, off);
      int oi = __shfl_xor(bi, off);
      if (op > bp || (op == bp && oi < bi)) {
        bp = op;
        bi = oi;
      }
    }
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

template <int EPL>
__global__ __launch_bounds__(256) void k_route(const uint16_t* __restrict__ logits, long long ld,
                                               int T, int E, int k, long long* __restrict__ idx64,
                                               int* __restrict__ idx32, uint16_t* __restrict__ w_out,
                                               int* __restrict__ counts) {
  int lane = threadIdx.x & 63;
  int t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t >= T) return;
  route_rows<EPL>(logits, ld, t, E, k, lane, idx64, idx32, w_out, nullptr, counts);
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

// ------------------------------------------------------------------- small fused path

// One workgroup: (optionally) route T rows, then count, scan, build the tile table
// and scatter the stable order. P = T * k <= kSmallMaxPairs, E <= kSmallMaxE.
template <int EPL>
__global__ __launch_bounds__(kSortThreads) void k_route_sort_small(
    const uint16_t* __restrict__ logits, long long ld, const int* __restrict__ ids32_in,
    const long long* __restrict__ ids64_in, int T, int E, int k, int bm, int has_shared,
    long long* __restrict__ idx64, int* __restrict__ idx32, uint16_t* __restrict__ w_out,
    int* __restrict__ counts_g, int* __restrict__ offsets_g, int* __restrict__ order,
    int* __restrict__ table, int MT) {
  __shared__ int keys[kSmallMaxPairs];
  __shared__ int hist[kSmallMaxE];
  __shared__ int offs[kSmallMaxE];
  __shared__ int wcnt[kSortWaves * kSmallMaxE];
  __shared__ int tmp[kSortWaves + 1];
  const int P = T * k;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int e = threadIdx.x; e < E; e += blockDim.x) hist[e] = 0;
  if (logits) {
    for (int t = wave; t < T; t += kSortWaves)
      route_rows<EPL>(logits, ld, t, E, k, lane, idx64, idx32, w_out, keys, nullptr);
  } else {
    for (int p = threadIdx.x; p < P; p += blockDim.x) {
      long long v = ids64_in ? ids64_in[p] : (long long)ids32_in[p];
      keys[p] = (int)(v < 0 ? 0 : (v >= E ? E - 1 : v));  // clamp as batched_mm does
    }
  }
  __syncthreads();
  for (int p = threadIdx.x; p < P; p += blockDim.x) atomicAdd(&hist[keys[p]], 1);
  __syncthreads();
  build_table(hist, E, P, T, bm, has_shared, offs, counts_g, offsets_g, table, MT, tmp);
  const int nbits = E > 1 ? 32 - __clz(E - 1) : 1;
  for (int c0 = 0; c0 < P; c0 += blockDim.x) {
    int p = c0 + threadIdx.x;
    bool valid = p < P;
    int key = valid ? keys[p] : 0;
    int rank = block_stable_rank(key, valid, E, nbits, wcnt);
    if (valid) order[offs[key] + rank] = p;
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
      int s = 0;
      for (int v = 0; v < kSortWaves; ++v) s += wcnt[v * E + e];
      offs[e] += s;
    }
    __syncthreads();
  }
}

// -------------------------------------------------------------------- multi-block path

__device__ __forceinline__ int load_key(const int* ids32, const long long* ids64, long long p,
                                        int E) {
  long long v = ids64 ? ids64[p] : (long long)ids32[p];
  return (int)(v < 0 ? 0 : (v >= E ? E - 1 : v));
}

// Per-block histograms: bcnt[b * E + e].
__global__ __launch_bounds__(kSortThreads) void k_sort_count(const int* __restrict__ ids32,
                                                             const long long* __restrict__ ids64,
                                                             int P, int E,
                                                             int* __restrict__ bcnt) {
  __shared__ int hist[kMaxE];
  for (int e = threadIdx.x; e < E; e += blockDim.x) hist[e] = 0;
  __syncthreads();
  long long p = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (p < P) atomicAdd(&hist[load_key(ids32, ids64, p, E)], 1);
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x) bcnt[(long long)blockIdx.x * E + e] = hist[e];
}

// One workgroup: per-expert totals, offsets, the tile table, and bcnt turned into each
// block's first sorted row per expert.
__global__ __launch_bounds__(kSortThreads) void k_sort_scan(int* __restrict__ bcnt, int nblocks,
                                                            int P, int T, int E, int bm,
                                                            int has_shared, int* __restrict__ counts_g,
                                                            int* __restrict__ offsets_g,
                                                            int* __restrict__ table, int MT) {
  __shared__ int hist[kMaxE];
  __shared__ int offs[kMaxE];
  __shared__ int tmp[kSortWaves + 1];
  int e = threadIdx.x;
  if (e < E) {
    int acc = 0;
    for (int b = 0; b < nblocks; ++b) {
      int c = bcnt[(long long)b * E + e];
      bcnt[(long long)b * E + e] = acc;
      acc += c;
    }
    hist[e] = acc;
  }
  __syncthreads();
  build_table(hist, E, P, T, bm, has_shared, offs, counts_g, offsets_g, table, MT, tmp);
  if (e < E) {
    int o = offs[e];
    for (int b = 0; b < nblocks; ++b) bcnt[(long long)b * E + e] += o;
  }
}

__global__ __launch_bounds__(kSortThreads) void k_sort_scatter(const int* __restrict__ ids32,
                                                               const long long* __restrict__ ids64,
                                                               int P, int E,
                                                               const int* __restrict__ bbase,
                                                               int* __restrict__ order) {
  __shared__ int wcnt[kSortWaves * kMaxE];
  long long p = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  bool valid = p < P;
  int key = valid ? load_key(ids32, ids64, p, E) : 0;
  const int nbits = E > 1 ? 32 - __clz(E - 1) : 1;
  int rank = block_stable_rank(key, valid, E, nbits, wcnt);
  if (valid) order[bbase[(long long)blockIdx.x * E + key] + rank] = (int)p;
}

// ---------------------------------------------------------------------- host launchers

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

hipError_t launch_route(const uint16_t* logits, long long ld, int T, int E, int k, long long* idx64,
                        int* idx32, uint16_t* w_out, int* counts, hipStream_t s) {
  if (T <= 0) return hipSuccess;
  dim3 grid((T + 3) / 4), block(256);
#define L(EPL) hipLaunchKernelGGL(k_route<EPL>, grid, block, 0, s, logits, ld, T, E, k, idx64, idx32, w_out, counts)
  MOE_EPL_DISPATCH(E, L);
#undef L
  return hipGetLastError();
}

size_t sort_scratch_bytes(int P, int E) {
  if (P <= kSmallMaxPairs && E <= kSmallMaxE) return 0;
  size_t nb = (P + kSortThreads - 1) / kSortThreads;
  return nb * (size_t)E * sizeof(int);
}

bool sort_uses_small(int P, int E) { return P <= kSmallMaxPairs && E <= kSmallMaxE; }

// Route (when logits) and sort. ids (int32 or int64) are read when logits is null,
// written (idx64/idx32/w_out) when logits is given.
hipError_t launch_route_sort(const uint16_t* logits, long long ld, const int* ids32_in,
                             const long long* ids64_in, int T, int E, int k, int bm, int has_shared,
                             long long* idx64, int* idx32, uint16_t* w_out, int* counts,
                             int* offsets, int* order, int* table, int MT, int* scratch,
                             hipStream_t s) {
  const int P = T * k;
  if (sort_uses_small(P, E)) {
#define L(EPL)                                                                                 \
  hipLaunchKernelGGL(k_route_sort_small<EPL>, dim3(1), dim3(kSortThreads), 0, s, logits, ld,  \
                     ids32_in, ids64_in, T, E, k, bm, has_shared, idx64, idx32, w_out, counts, \
                     offsets, order, table, MT)
    MOE_EPL_DISPATCH(E, L);
#undef L
    return hipGetLastError();
  }
  const int* k32 = ids32_in;
  const long long* k64 = ids64_in;
  if (logits) {
    hipError_t err = launch_route(logits, ld, T, E, k, idx64, idx32, w_out, nullptr, s);
    if (err != hipSuccess) return err;
    if (idx32) {
      k32 = idx32;
      k64 = nullptr;
    } else {
      k32 = nullptr;
      k64 = idx64;
    }
  }
  int nb = (P + kSortThreads - 1) / kSortThreads;
  hipLaunchKernelGGL(k_sort_count, dim3(nb), dim3(kSortThreads), 0, s, k32, k64, P, E, scratch);
  hipLaunchKernelGGL(k_sort_scan, dim3(1), dim3(kSortThreads), 0, s, scratch, nb, P, T, E, bm,
                     has_shared, counts, offsets, table, MT);
  hipLaunchKernelGGL(k_sort_scatter, dim3(nb), dim3(kSortThreads), 0, s, k32, k64, P, E, scratch,
                     order);
  return hipGetLastError();
}

}  // namespace moe
