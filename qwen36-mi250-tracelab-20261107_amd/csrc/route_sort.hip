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
#include "route_sort_dev.h"

namespace moe {

// ---------------------------------------------------------------------------- routing

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

// Routing from the router's four fp32 K-quarter partial sums (k_router_part): the logits
// are bf16(((s0 + s1) + s2) + s3), the bits every router kernel gives; each token's row is
// written to `logits` (all n_pack entries) and routed from registers.
template <int EPL>
__global__ __launch_bounds__(256) void k_route_part(const float* __restrict__ part, int T,
                                                    int n_pack, int E, int k,
                                                    uint16_t* __restrict__ logits,
                                                    long long* __restrict__ idx64,
                                                    int* __restrict__ idx32,
                                                    uint16_t* __restrict__ w_out) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t >= T) return;
  const long long qs = (long long)T * n_pack;  // stride between quarters
  const float* p = part + (long long)t * n_pack;
  uint16_t* lrow = logits + (long long)t * n_pack;
  auto logit = [&](int e) __attribute__((always_inline)) {
    return f2bf_bits(((p[e] + p[qs + e]) + p[2 * qs + e]) + p[3 * qs + e]);
  };
  uint16_t raw[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane + kWave * i;
    raw[i] = e < n_pack ? logit(e) : 0;
    if (e < n_pack) lrow[e] = raw[i];
  }
  for (int e = kWave * EPL + lane; e < n_pack; e += kWave) lrow[e] = logit(e);
  int my_i;
  float my_w;
  route_row_raw<EPL>(raw, E, k, lane, my_i, my_w);
  if (lane < k) {
    const long long pidx = (long long)t * k + lane;
    if (idx64) idx64[pidx] = my_i;
    if (idx32) idx32[pidx] = my_i;
    if (w_out) w_out[pidx] = f2bf_bits(my_w);
  }
}

// ------------------------------------------------------------------- small fused path

template <int EPL>
__global__ __launch_bounds__(kSortThreads) void k_route_sort_small(
    const uint16_t* __restrict__ logits, long long ld, const int* __restrict__ ids32_in,
    const long long* __restrict__ ids64_in, int T, int E, int k, int bm, int has_shared,
    long long* __restrict__ idx64, int* __restrict__ idx32, uint16_t* __restrict__ w_out,
    int* __restrict__ counts_g, int* __restrict__ offsets_g, int* __restrict__ order,
    int* __restrict__ table, int MT) {
  __shared__ SortLds L;
  route_sort_block<EPL>(logits, ld, ids32_in, ids64_in, T, E, k, bm, has_shared, idx64, idx32,
                        w_out, counts_g, offsets_g, order, table, MT, L);
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
  // Per-expert exclusive scan over the blocks. The block counts are read in groups of 16
  // whose loads are all in flight together (one memory round trip per group, not per block).
  constexpr int G = 16;
  int e = threadIdx.x;
  if (nblocks <= 2 * G) {
    // up to 32 blocks: one round trip, the counts kept in registers for the final bases
    int c[2 * G], base[2 * G];
    int acc = 0;
    if (e < E) {
#pragma unroll
      for (int i = 0; i < 2 * G; ++i) c[i] = i < nblocks ? bcnt[(long long)i * E + e] : 0;
#pragma unroll
      for (int i = 0; i < 2 * G; ++i) {
        base[i] = acc;
        acc += c[i];
      }
      hist[e] = acc;
    }
    __syncthreads();
    build_table(hist, E, P, T, bm, has_shared, offs, counts_g, offsets_g, table, MT, tmp);
    if (e < E) {
      const int o = offs[e];
#pragma unroll
      for (int i = 0; i < 2 * G; ++i)
        if (i < nblocks) bcnt[(long long)i * E + e] = base[i] + o;
    }
    return;
  }
  if (e < E) {
    int acc = 0;
    for (int b0 = 0; b0 < nblocks; b0 += G) {
      int c[G];
#pragma unroll
      for (int i = 0; i < G; ++i) c[i] = b0 + i < nblocks ? bcnt[(long long)(b0 + i) * E + e] : 0;
#pragma unroll
      for (int i = 0; i < G; ++i) {
        if (b0 + i < nblocks) bcnt[(long long)(b0 + i) * E + e] = acc;
        acc += c[i];
      }
    }
    hist[e] = acc;
  }
  __syncthreads();
  build_table(hist, E, P, T, bm, has_shared, offs, counts_g, offsets_g, table, MT, tmp);
  if (e < E) {
    const int o = offs[e];
    for (int b0 = 0; b0 < nblocks; b0 += G) {
      int c[G];
#pragma unroll
      for (int i = 0; i < G; ++i) c[i] = b0 + i < nblocks ? bcnt[(long long)(b0 + i) * E + e] : 0;
#pragma unroll
      for (int i = 0; i < G; ++i)
        if (b0 + i < nblocks) bcnt[(long long)(b0 + i) * E + e] = c[i] + o;
    }
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

hipError_t launch_route(const uint16_t* logits, long long ld, int T, int E, int k, long long* idx64,
                        int* idx32, uint16_t* w_out, int* counts, hipStream_t s) {
  if (T <= 0) return hipSuccess;
  dim3 grid((T + 3) / 4), block(256);
#define L(EPL) hipLaunchKernelGGL(k_route<EPL>, grid, block, 0, s, logits, ld, T, E, k, idx64, idx32, w_out, counts)
  MOE_EPL_DISPATCH(E, L);
#undef L
  return hipGetLastError();
}

hipError_t launch_route_part(const float* part, int T, int n_pack, int E, int k,
                             uint16_t* logits, long long* idx64, int* idx32, uint16_t* w_out,
                             hipStream_t s) {
  if (T <= 0) return hipSuccess;
  dim3 grid((T + 3) / 4), block(256);
#define L(EPL) hipLaunchKernelGGL(k_route_part<EPL>, grid, block, 0, s, part, T, n_pack, E, k, logits, idx64, idx32, w_out)
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

// Up to this many tokens the one-workgroup kernel also routes (fewer launches).
constexpr int kRouteSortFusedMaxTokens = 16;

// Route (when logits) and sort. ids (int32 or int64) are read when logits is null,
// written (idx64/idx32/w_out) when logits is given.
hipError_t launch_route_sort(const uint16_t* logits, long long ld, const int* ids32_in,
                             const long long* ids64_in, int T, int E, int k, int bm, int has_shared,
                             long long* idx64, int* idx32, uint16_t* w_out, int* counts,
                             int* offsets, int* order, int* table, int MT, int* scratch,
                             hipStream_t s) {
  const int P = T * k;
  if (logits && sort_uses_small(P, E) && T > kRouteSortFusedMaxTokens) {
    // one wave per token across many workgroups, then the one-workgroup sort: faster than
    // routing all tokens inside the sorting workgroup once there are more than a few
    hipError_t err = launch_route(logits, ld, T, E, k, idx64, idx32, w_out, nullptr, s);
    if (err != hipSuccess) return err;
    return launch_route_sort(nullptr, 0, idx32 ? idx32 : nullptr, idx32 ? nullptr : idx64, T, E,
                             k, bm, has_shared, nullptr, nullptr, nullptr, counts, offsets, order,
                             table, MT, scratch, s);
  }
  if (sort_uses_small(P, E)) {
    // one workgroup; a few tokens need few waves (fewer barriers to wait at)
    int need = P > E ? P : E;
    int threads = T > 16 ? kSortThreads : ((need + 63) / 64) * 64;
    if (threads > kSortThreads) threads = kSortThreads;
#define L(EPL)                                                                                 \
  hipLaunchKernelGGL(k_route_sort_small<EPL>, dim3(1), dim3(threads), 0, s, logits, ld,       \
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
