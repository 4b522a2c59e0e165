// Router logits of tiled batches (more than the decode path's few tokens) on gfx950
// (subsystem a1): logits[t, n] = bf16(x_t . w_pack[n]) with fp32 accumulation, the router
// F.linear of modeling_qwen3_5_moe.py:768-769 / engine/fast/model.py:1159 and the merged
// projection of engine/fast/prefill_kernels.py:91 (`project`, used at :693).
//
// Batch invariance. Every logit is summed in ONE fixed order whatever the batch size or
// the tile configuration: K (the hidden size) is split into four quarters, wave w of a
// workgroup sums quarter w with v_mfma_f32_16x16x32_bf16 k-steps of 32 in ascending order,
// and the four partial sums are added as ((s0 + s1) + s2) + s3. The tile shape (how many
// 16-token and 16-row blocks a wave holds) only changes which outputs a workgroup makes, not
// how any one of them is summed, so the configuration can follow the batch size and a
// token's logits (hence its routing) never depend on the tokens batched with it.
//
// Two kernels give those bits:
// * k_router_gemm (up to ~1k tokens): K split over the 4 waves of a workgroup. No operand is
//   shared between its waves (each needs its own K quarter of both), so both go straight
//   from global memory into registers in the MFMA operand layout (lane l: row l % 16,
//   k = 8 (l / 16) .. + 8; 64 contiguous bytes of each of 16 rows per load instruction), R
//   k-steps in flight per wave; LDS holds only the final reduction.
// * k_router_dma (from 768 tokens): 64 tokens x 64 rows per workgroup, both operands staged
//   by global -> LDS DMA and shared by 4 waves; each wave runs the whole K, restarting its
//   accumulator at every quarter and folding it into a running total, which reproduces
//   ((s0 + s1) + s2) + s3 bit for bit with a quarter of the operand traffic of the split
//   kernel (16.1 against 20.7 µs for a register-staged form of the same tiles at 4096
//   tokens, 12.7 against 14.8 at 768).
// Workgroups of one token tile get ids 8 apart so they run on one XCD and share the tile's
// token rows in its L2 (the router rows, 1.25 MiB, stay in every XCD's L2).
#include <stdio.h>
#include <stdlib.h>

#include <mutex>

#include "moe_common.h"
#include "lds_dma.h"

namespace moe {

namespace {

constexpr int kRouterSplit = 4;  // K quarters = waves per workgroup (fixes the sum order)
constexpr int kXcdsR = 8;
constexpr int kRouterTilesFrom = 768;  // tokens from which the LDS-tiled kernel runs

struct RouterArgs {
  const uint16_t* x;  // [T, H]
  const uint16_t* w;  // [n_pack, H]
  uint16_t* out;      // [T, n_pack]
  int T, H, n_pack;
  int ntiles, nrg;    // token tiles, row groups
  int xcd_map;        // workgroups of one token tile 8 ids apart (at least 8 tiles)
};

// TB 16-token blocks x RB 16-row blocks per wave; R k-steps of loads in flight.
template <int TB, int RB, int R>
__global__ __launch_bounds__(64 * kRouterSplit) void k_router_gemm(RouterArgs a) {
  __shared__ f32x4_t red[kRouterSplit - 1][TB * RB][kWave];
  int tile, rg;
  if (a.xcd_map) {
    const int xcd = blockIdx.x & (kXcdsR - 1);
    const int j = blockIdx.x / kXcdsR;
    tile = (j / a.nrg) * kXcdsR + xcd;
    rg = j - (j / a.nrg) * a.nrg;
    if (tile >= a.ntiles) return;
  } else {
    tile = blockIdx.x / a.nrg;
    rg = blockIdx.x - tile * a.nrg;
  }

  const int lane = threadIdx.x & 63;
  const int wk = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lr = lane & 15;
  const int q = lane >> 4;
  const int Kq = a.H / kRouterSplit;
  const int kbeg = wk * Kq;
  const int nst = Kq / 32;
  const int t0 = tile * 16 * TB;
  const int n0 = rg * 16 * RB;
  // blocks that hold real rows / tokens (wave-uniform: n_pack is a multiple of 16)
  const int nrb = __builtin_amdgcn_readfirstlane(min(RB, (a.n_pack - n0) / 16));
  const int ntb = __builtin_amdgcn_readfirstlane(min(TB, (a.T - t0 + 15) / 16));

  const uint16_t* wa[RB];
  const uint16_t* xb[TB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
    wa[rb] = a.w + (long long)min(n0 + rb * 16 + lr, a.n_pack - 1) * a.H + kbeg + q * 8;
#pragma unroll
  for (int tb = 0; tb < TB; ++tb)
    xb[tb] = a.x + (long long)min(t0 + tb * 16 + lr, a.T - 1) * a.H + kbeg + q * 8;

  uint4 ra[R][RB], rx[R][TB];
  auto issue = [&](int slot, int s) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
      if (rb < nrb) ra[slot][rb] = ld16(wa[rb] + s * 32);
#pragma unroll
    for (int tb = 0; tb < TB; ++tb)
      if (tb < ntb) rx[slot][tb] = ld16(xb[tb] + s * 32);
  };
#pragma unroll
  for (int s = 0; s < R; ++s)
    if (s < nst) issue(s, s);

  f32x4_t acc[TB][RB];
#pragma unroll
  for (int tb = 0; tb < TB; ++tb)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[tb][rb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int s0 = 0; s0 < nst; s0 += R) {
#pragma unroll
    for (int c = 0; c < R; ++c) {
      const int s = s0 + c;
      if (s >= nst) break;
#pragma unroll
      for (int tb = 0; tb < TB; ++tb)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          if (tb < ntb && rb < nrb) acc[tb][rb] = mfma16x16x32(ra[c][rb], rx[c][tb], acc[tb][rb]);
      if (s + R < nst) issue(c, s + R);
    }
  }

  // ((s0 + s1) + s2) + s3 in wave order
  if (wk > 0) {
#pragma unroll
    for (int tb = 0; tb < TB; ++tb)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) red[wk - 1][tb * RB + rb][lane] = acc[tb][rb];
  }
  __syncthreads();
  if (wk > 0) return;
#pragma unroll
  for (int v = 0; v < kRouterSplit - 1; ++v)
#pragma unroll
    for (int tb = 0; tb < TB; ++tb)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) acc[tb][rb] += red[v][tb * RB + rb][lane];

  // lane (q, j = lr) holds rows 4q .. 4q + 3 of token column j of each block
#pragma unroll
  for (int tb = 0; tb < TB; ++tb) {
    const int t = t0 + tb * 16 + lr;
    if (tb >= ntb || t >= a.T) continue;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      if (rb >= nrb) break;
      const int n = n0 + rb * 16 + 4 * q;
      const f32x4_t v = acc[tb][rb];
      *reinterpret_cast<uint2*>(a.out + (long long)t * a.n_pack + n) =
          make_uint2(pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]));
    }
  }
}

// k_router_part: the split kernel's work with one wave per workgroup, i.e. one K quarter
// of one 16-token x 16-row block per workgroup (four times as many workgroups, each a
// quarter of the chain), its fp32 partial sum stored to part[q][t][n]. The caller sums the
// quarters as ((s0 + s1) + s2) + s3 and rounds (k_route_part), which gives the same logits
// as k_router_gemm. For small batches, where k_router_gemm has too few workgroups to fill
// the GPU.
template <int NST>
__global__ __launch_bounds__(64) void k_router_part(RouterArgs a, float* __restrict__ part) {
  // the four quarter workgroups of a block get ids 8 apart: one XCD fetches the block's rows
  // whole (as the four waves of a k_router_gemm workgroup do)
  const int xcd = blockIdx.x & (kXcdsR - 1);
  const int i = blockIdx.x / kXcdsR;
  const int wk = i & (kRouterSplit - 1);
  const int blk = (i / kRouterSplit) * kXcdsR + xcd;
  if (blk >= a.ntiles * a.nrg) return;
  const int tile = blk / a.nrg;
  const int rg = blk - tile * a.nrg;
  const int lane = threadIdx.x;
  const int lr = lane & 15;
  const int q = lane >> 4;
  const int kbeg = wk * NST * 32;  // the quarter: NST k-steps of 32
  const int t0 = tile * 16;
  const int n0 = rg * 16;
  const uint16_t* wa = a.w + (long long)(n0 + lr) * a.H + kbeg + q * 8;
  const uint16_t* xb = a.x + (long long)min(t0 + lr, a.T - 1) * a.H + kbeg + q * 8;
  // the whole quarter's operands in flight at once
  uint4 ra[NST], rx[NST];
#pragma unroll
  for (int s = 0; s < NST; ++s) {
    ra[s] = ld16(wa + s * 32);
    rx[s] = ld16(xb + s * 32);
  }
  f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < NST; ++s) acc = mfma16x16x32(ra[s], rx[s], acc);
  // lane (q, j = lr) holds rows 4q .. 4q + 3 of token column j
  const int t = t0 + lr;
  if (t < a.T)
    *reinterpret_cast<f32x4_t*>(part + ((long long)wk * a.T + t) * a.n_pack + n0 + 4 * q) = acc;
}

// ------------------------------------------------------------------ LDS-tiled form

constexpr int kTT = 64;                 // tokens per tile
constexpr int kTN = 64;                 // router rows per tile
constexpr int kTRows = kTT + kTN;       // staged rows per chunk (tokens, then router rows)

// k_router_dma: 64 tokens x 64 router rows per workgroup, both operands staged by global ->
// LDS DMA (global_load_lds_dwordx4: no registers on the way) and shared by 4 waves (2 x 2
// blocks of 16 each), in a ring of S stages, chunk d + S - 1 requested while chunk d is
// multiplied. Each wave runs the whole K, restarting its accumulator at every quarter and
// folding it into a running total, which reproduces ((s0 + s1) + s2) + s3 bit for bit. Wave w's DMA load i
// fills the 4-row group w + 4 i of a stage (1 KiB: 4 rows x 256 bytes), lane l writing
// physical unit l & 15 of row l >> 4 of the group with logical unit (l & 15) ^ (row & 15):
// the XOR order that keeps the fragment reads (16 rows, one logical unit) bank-conflict
// free. Fragments are read by inline asm with explicit waits (lds_dma.h).
template <int S>
__global__ __launch_bounds__(256) void k_router_dma(RouterArgs a) {
  constexpr int KC = 128;                       // k per chunk: 256 bytes of each row
  constexpr int kUnits = KC / 8;                // 16-byte units per staged row
  constexpr int kRowBytes = KC * 2;
  constexpr int kStage = kTRows * kRowBytes;    // 32 KiB
  constexpr int kGroups = kTRows / 4;           // 4-row DMA groups per chunk: 32
  constexpr int kLoads = kGroups / 4;           // per wave and chunk: 8
  static_assert(kLoads * 4 == kGroups && (kLoads * (S - 2)) <= 12, "wait_loads range");
  extern __shared__ uint4 smem[];
  int tile, rg;
  if (a.xcd_map) {
    const int xcd = blockIdx.x & (kXcdsR - 1);
    const int j = blockIdx.x / kXcdsR;
    tile = (j / a.nrg) * kXcdsR + xcd;
    rg = j - (j / a.nrg) * a.nrg;
    if (tile >= a.ntiles) return;
  } else {
    tile = blockIdx.x / a.nrg;
    rg = blockIdx.x - tile * a.nrg;
  }
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wt = wave & 1, wn = wave >> 1;
  const int lr = lane & 15, kq = lane >> 4;
  const int t0 = tile * kTT, n0 = rg * kTN;

  // DMA sources: group g = wave + 4 i, row 4 g + (lane >> 4) (tokens, then router rows)
  const uint16_t* src[kLoads];
#pragma unroll
  for (int i = 0; i < kLoads; ++i) {
    const int row = (wave + 4 * i) * 4 + (lane >> 4);
    const int lu = (lane & 15) ^ (row & (kUnits - 1));
    src[i] = row < kTT ? a.x + (long long)min(t0 + row, a.T - 1) * a.H + lu * 8
                       : a.w + (long long)min(n0 + row - kTT, a.n_pack - 1) * a.H + lu * 8;
  }
  char* lds = reinterpret_cast<char*>(smem);
  auto issue = [&](int d) __attribute__((always_inline)) {
    char* st = lds + (d % S) * kStage;
#pragma unroll
    for (int i = 0; i < kLoads; ++i)
      __builtin_amdgcn_global_load_lds(src[i] + d * KC, st + (wave + 4 * i) * 1024, 16, 0, 0);
  };
  const uint32_t lbase = lds_addr(lds);
  // this lane's fragment rows: router rows wn * 32 + r * 16 + lr, tokens wt * 32 + b * 16 + lr
  const uint32_t arow0 = (uint32_t)((kTT + wn * 32 + lr) * kRowBytes);
  const uint32_t brow0 = (uint32_t)((wt * 32 + lr) * kRowBytes);

  f32x4_t acc[2][2], tot[2][2];  // [token block][row block]
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int r = 0; r < 2; ++r) acc[b][r] = tot[b][r] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int nd = a.H / KC;
  const int per_q = nd / kRouterSplit;
#pragma unroll
  for (int c = 0; c < S - 1; ++c)
    if (c < nd) issue(c);
  for (int d = 0; d < nd; ++d) {
    // chunk d: younger than it are chunks d + 1 .. d + S - 2 where issued
    wait_loads(kLoads * max(0, min(S - 2, nd - 1 - d)));
    __builtin_amdgcn_s_barrier();  // chunk d visible; the slot of chunk d - 1 free
    if (d + S - 1 < nd) issue(d + S - 1);
    const uint32_t st = lbase + (d % S) * kStage;
#pragma unroll
    for (int h = 0; h < KC / 32; ++h) {
      // logical unit h * 4 + kq of each row, at its physical position
      const uint32_t ua = (uint32_t)((((h * 4 + kq) ^ (lr & (kUnits - 1)))) * 16);
      u32x4v fa[2], fb[2];
      fa[0] = lds_read_frag<0>(st + arow0 + ua);
      fa[1] = lds_read_frag<16 * kRowBytes>(st + arow0 + ua);
      fb[0] = lds_read_frag<0>(st + brow0 + ua);
      fb[1] = lds_read_frag<16 * kRowBytes>(st + brow0 + ua);
      lds_frags_ready();
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        after_wait(fa[i]);
        after_wait(fb[i]);
      }
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 2; ++r) acc[b][r] = mfma_frag(fa[r], fb[b], acc[b][r]);
    }
    if ((d + 1) % per_q == 0) {  // end of a K quarter: total = ((s0 + s1) + s2) + s3
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          tot[b][r] = d + 1 == per_q ? acc[b][r] : tot[b][r] + acc[b][r];
          acc[b][r] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        }
    }
  }
  // lane (q = kq, j = lr) holds rows 4q .. 4q + 3 of token column j of each block
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int t = t0 + wt * 32 + b * 16 + lr;
    if (t >= a.T) continue;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int n = n0 + wn * 32 + r * 16 + 4 * kq;
      if (n >= a.n_pack) continue;
      const f32x4_t v = tot[b][r];
      *reinterpret_cast<uint2*>(a.out + (long long)t * a.n_pack + n) =
          make_uint2(pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]));
    }
  }
}

struct RCfg {
  int tb, rb, r;
};

// Tile configuration of the split kernel by batch size (it does not change any logit's
// bits). Measured per call at H=2048, n_pack=320 (8 launches graph-replayed): T <= 128
// (1,1,4) 6.1-6.2 µs; 256 (2,1,8) 9.3; 512 (2,2,4) 11.4; 1024 (4,2,4) 15.9 (the tiled
// kernel, 128-k chunks: 14.7 from ~1k tokens; 20.5 at 4096 against 39.7 here).
RCfg router_cfg(int T) {
  if (T <= 128) return {1, 1, 4};
  if (T <= 384) return {2, 1, 8};
  return {2, 2, 4};
}

}  // namespace

bool router_gemm_fits(int H, int n_pack) { return H % (32 * kRouterSplit) == 0 && n_pack % 16 == 0; }

// The block forward's router for T tokens: k_router_part + k_route_part where the routing is
// a launch of its own anyway (more than 16 tokens) and the split kernel has few workgroups.
// Measured per layer (8 layers cycled, uniform routing): 17 / 32 / 64 / 128 / 256 tokens
// 154.0 / 207.8 / 263.9 / 297.8 / 318.9 µs against 155.4 / 209.8 / 265.6 / 298.8 / 320.6
// with k_router_gemm then k_route; level at 512 tokens (372.8 against 371.9), slower at 767
// (390.1 against 386.2). At C3 the router launch takes 4.8 µs against 7.7.
bool router_part_takes(int T, int H, int n_pack) {
  const int nst = H / (32 * kRouterSplit);
  return router_gemm_fits(H, n_pack) && (nst == 4 || nst == 8 || nst == 16) && T > 16 &&
         T <= 256;
}

hipError_t launch_router_part(const void* x, int T, int H, const void* w_pack, int n_pack,
                              float* part, hipStream_t st) {
  if (!router_gemm_fits(H, n_pack)) return hipErrorInvalidValue;
  if (T <= 0) return hipSuccess;
  RouterArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.w = static_cast<const uint16_t*>(w_pack);
  a.T = T;
  a.H = H;
  a.n_pack = n_pack;
  a.ntiles = (T + 15) / 16;
  a.nrg = n_pack / 16;
  const long long nblk = (long long)a.ntiles * a.nrg;
  const long long grid = (nblk + kXcdsR - 1) / kXcdsR * kXcdsR * kRouterSplit;
  if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
  switch (H / (32 * kRouterSplit)) {
    case 4:
      hipLaunchKernelGGL(k_router_part<4>, dim3((unsigned)grid), dim3(64), 0, st, a, part);
      break;
    case 8:
      hipLaunchKernelGGL(k_router_part<8>, dim3((unsigned)grid), dim3(64), 0, st, a, part);
      break;
    case 16:
      hipLaunchKernelGGL(k_router_part<16>, dim3((unsigned)grid), dim3(64), 0, st, a, part);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_router_gemm(const void* x, int T, int H, const void* w_pack, int n_pack,
                              void* logits, hipStream_t st) {
  if (!router_gemm_fits(H, n_pack)) return hipErrorInvalidValue;
  if (T <= 0) return hipSuccess;
  RouterArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.w = static_cast<const uint16_t*>(w_pack);
  a.out = static_cast<uint16_t*>(logits);
  a.T = T;
  a.H = H;
  a.n_pack = n_pack;
  if (T >= kRouterTilesFrom && H % (kRouterSplit * 128) == 0) {
    a.ntiles = (T + kTT - 1) / kTT;
    a.nrg = (n_pack + kTN - 1) / kTN;
    a.xcd_map = a.ntiles >= kXcdsR;
    const long long grid = a.xcd_map
                               ? (long long)((a.ntiles + kXcdsR - 1) / kXcdsR) * kXcdsR * a.nrg
                               : (long long)a.ntiles * a.nrg;
    if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
    constexpr int kStages = 2;
    const int bytes = kStages * kTRows * 256;
    static std::mutex mu;
    static uint64_t done = 0;  // bit d: the LDS limit is raised on device d
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return err;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    {
      std::lock_guard<std::mutex> lock(mu);
      if (!(done >> dev & 1)) {
        err = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_router_dma<kStages>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
        if (err != hipSuccess) return err;
        done |= uint64_t(1) << dev;
      }
    }
    hipLaunchKernelGGL(k_router_dma<kStages>, dim3((unsigned)grid), dim3(256), bytes, st, a);
    return hipGetLastError();
  }
  const RCfg c = router_cfg(T);
  a.ntiles = (T + 16 * c.tb - 1) / (16 * c.tb);
  a.nrg = (n_pack + 16 * c.rb - 1) / (16 * c.rb);
  a.xcd_map = a.ntiles >= kXcdsR;
  const long long grid = a.xcd_map
                             ? (long long)((a.ntiles + kXcdsR - 1) / kXcdsR) * kXcdsR * a.nrg
                             : (long long)a.ntiles * a.nrg;
  if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
  const dim3 block(64 * kRouterSplit);
#define RL(TB, RB, RR)                                                                   \
  if (c.tb == TB && c.rb == RB && c.r == RR) {                                           \
    hipLaunchKernelGGL((k_router_gemm<TB, RB, RR>), dim3((unsigned)grid), block, 0, st, a); \
    return hipGetLastError();                                                            \
  }
  RL(1, 1, 4)
  RL(2, 1, 8)
  RL(2, 2, 4)
#undef RL
  return hipErrorInvalidValue;
}

}  // namespace moe
