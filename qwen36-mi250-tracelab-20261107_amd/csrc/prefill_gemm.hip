// Grouped MFMA GEMM for prefill-sized batches on gfx950 (subsystems a8, a9, a6).
//
// Same contract as k_expert_gemm (expert_gemm.hip) and the reference's grouped kernels
// (engine/fast/moe_prefill.py:156-257): for a tile of up to 256 sorted rows of ONE expert,
//   SWIGLU: act[r, n]       = bf16(bf16(silu(bf16 g)) * bf16 u)
//   PLAIN:  out[orow(r), n] = bf16(act_or_x[r] . W[e, n])
// but tiled for ~128 tokens per expert: a workgroup computes 256 weight rows x 256 tokens
// with both operands staged in LDS, so every weight byte read from HBM feeds every token of
// the tile and every token byte feeds 256 weight rows.
//
// Layout. 8 waves: wave (wm, wn) owns weight rows [64 wm, 64 wm + 64) and the 16-token
// blocks 2 b + wn (b < 8) of the tile (alternating, so a part-filled tile keeps both token
// waves busy): 4 x 8 blocks of v_mfma_f32_16x16x32_bf16, 128 accumulator registers. SWIGLU
// puts gate rows in blocks 0-1 and the matching up rows in blocks 2-3 of a wave, so the
// epilogue pairs them in registers.
//
// Pipeline. K runs in DMA chunks of 64 (128 bytes of each row). A chunk of one operand is
// 32 groups of 8 rows x 128 B; each group is one 1 KiB global -> LDS DMA load of a wave
// (global_load_lds_dwordx4: no registers on the way), lane l writing physical 16-byte unit
// l & 7 of row l >> 3, which holds logical unit (l & 7) ^ row, so the MFMA fragment reads
// (16 rows x one logical unit = one 1 KiB LDS read per 16 x 32 fragment) are bank-conflict
// free. Weight ring of 3 stages (chunk c + 2 requested while c is multiplied), token-row
// ring of 2 (c + 1): 160 KiB. The fragments of the next k-step (32) are read while the
// current one is multiplied. The fragment reads are issued by inline asm with explicit
// lgkmcnt waits and the stages are fenced by explicit vmcnt waits, because the compiler's
// own waits would drain every outstanding DMA load before each LDS read.
#include <stdint.h>
#include <stdlib.h>

#include <mutex>

#include "moe_common.h"
#include "expert_gemm.h"
#include "lds_dma.h"

namespace moe {

namespace {
constexpr int PBM = 256;                          // tokens per tile
constexpr int PBN = 256;                          // weight rows per workgroup
constexpr int PKC = 32;                           // K elements per MFMA k-step
constexpr int DKC = 64;                           // K elements per DMA chunk (128-byte rows)
constexpr int kRowBytes = DKC * 2;                // 128
constexpr int kBlkBytes = 16 * kRowBytes;         // a 16-row fragment block: 2 KiB
constexpr int kOpStage = 256 * kRowBytes;         // one operand of one chunk: 32 KiB
constexpr int kStagesA = 3, kAheadA = 2;          // weight ring: chunk d + 3 loads at step d
constexpr int kStagesB = 2, kAheadB = 1;          // token-row ring: chunk d + 2
constexpr int kLdsBytes = (kStagesA + kStagesB) * kOpStage;  // 160 KiB
constexpr int kThreads = 512;
constexpr int kXcds = 8;                          // XCDs of an MI355X (round-robin dispatch)
// Weight rows are read once per tile: their DMA loads are non-temporal (cache policy NT), so
// they do not displace the token rows the tile's other workgroups read again, or the pair
// outputs the combine reads next (C4 530 against 547 µs per layer; the token rows loaded
// non-temporal as well measured 552).
constexpr int kWeightCachePolicy = 2;
constexpr int kGroups = 256 / 8;                  // 8-row DMA groups per operand and chunk
constexpr int kLoadsPerWave = kGroups / (kThreads / 64);  // per operand and chunk: 4
static_assert(kLoadsPerWave == 4, "wait_loads counts 4 loads per operand per chunk");
static_assert(kAheadA <= kStagesA - 1 && kAheadB <= kStagesB - 1, "ring slots reused early");
}  // namespace

// MFMA fragments of one chunk for a wave: 4 weight-row blocks, 8 token blocks.
struct Frags {
  u32x4v a[4], b[8];
};

// Issue the wave's 12 fragment reads of one k-step from the A / B stages at astage /
// bstage (which include this lane's offset for the k-step); they complete at frags_ready.
__device__ __forceinline__ void read_frags(uint32_t astage, uint32_t bstage, int wm, int wn,
                                           Frags& f) {
  const uint32_t abase = astage + wm * 4 * kBlkBytes;
  const uint32_t bbase = bstage + wn * kBlkBytes;
  f.a[0] = lds_read_frag<0 * kBlkBytes>(abase);
  f.a[1] = lds_read_frag<1 * kBlkBytes>(abase);
  f.a[2] = lds_read_frag<2 * kBlkBytes>(abase);
  f.a[3] = lds_read_frag<3 * kBlkBytes>(abase);
  f.b[0] = lds_read_frag<0 * kBlkBytes>(bbase);
  f.b[1] = lds_read_frag<2 * kBlkBytes>(bbase);
  f.b[2] = lds_read_frag<4 * kBlkBytes>(bbase);
  f.b[3] = lds_read_frag<6 * kBlkBytes>(bbase);
  f.b[4] = lds_read_frag<8 * kBlkBytes>(bbase);
  f.b[5] = lds_read_frag<10 * kBlkBytes>(bbase);
  f.b[6] = lds_read_frag<12 * kBlkBytes>(bbase);
  f.b[7] = lds_read_frag<14 * kBlkBytes>(bbase);
}
__device__ __forceinline__ void frags_ready(Frags& f) {
  lds_frags_ready();
#pragma unroll
  for (int a = 0; a < 4; ++a) after_wait(f.a[a]);
#pragma unroll
  for (int b = 0; b < 8; ++b) after_wait(f.b[b]);
}
// MFMAs of the wave's first nb token blocks (nb wave-uniform: scalar branches).
__device__ __forceinline__ void mma_frags(const Frags& f, int nb, f32x4_t (&acc)[4][8]) {
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    if (b >= nb) break;
#pragma unroll
    for (int a = 0; a < 4; ++a) acc[a][b] = mfma_frag(f.a[a], f.b[b], acc[a][b]);
  }
}

template <int MODE>
__global__ __launch_bounds__(kThreads, 1) void k_prefill_gemm(GemmArgs args) {
  extern __shared__ uint4 smem[];  // A ring [kStagesA][16][1 KiB], B ring [kStagesB][16][1 KiB]

  // XCD-aware order: workgroup b runs on XCD b % 8, so the nrb workgroups of one tile get
  // ids 8 apart (same XCD, dispatched together) and share the tile's token rows in that
  // XCD's L2 instead of fetching them once per XCD.
  const int nrb = args.nrb;
  const int xcd = blockIdx.x & (kXcds - 1);
  const int j = blockIdx.x / kXcds;
  int tile = (j / nrb) * kXcds + xcd;
  const int rb = j - (j / nrb) * nrb;
  if (tile >= args.MTgrid) return;
  int e, r0, r1;
  if (args.table) {
    const int ntiles = args.table[3 * args.MT];
    if (tile >= ntiles) return;
    if (args.shared_first > 0) {
      // the shared expert's tiles (the table's last ones, whole 256-token tiles, the longest
      // workgroups) are dispatched first, the routed tiles fill in behind them
      const int ns = min(args.shared_first, ntiles);
      tile = tile < ns ? ntiles - ns + tile : tile - ns;
    }
    e = args.table[tile];
    r0 = args.table[args.MT + tile];
    // the table holds the expert's end row; this tile is its next PBM rows at most (the
    // token-row ring stages hold PBM rows)
    r1 = min(args.table[2 * args.MT + tile], r0 + PBM);
  } else {
    e = args.E;
    r0 = args.P + tile * PBM;
    if (r0 >= args.P + args.T) return;
    r1 = min(r0 + PBM, args.P + args.T);
  }
  const bool routed = e < args.E;
  const GemmOperand& op = routed ? args.op[0] : args.op[1];
  constexpr int kOutPerWG = MODE == kModeSwiglu ? PBN / 2 : PBN;
  if (rb * kOutPerWG >= op.N) return;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar)
  const int wm = wave & 3;   // weight-row group (64 rows)
  const int wn = wave >> 2;  // token-block parity
  const int lr = lane & 15;
  const int kq = lane >> 4;
  const int ntok = r1 - r0;

  // ---- DMA sources. A chunk of one operand is 256 rows x 128 B (64 k); each load of a wave
  // fills one 8-row group (1 KiB, 128 contiguous bytes of each row), the wave's groups being
  // wave + 8 i (i < 4). Lane l fills physical unit l & 7 of row l >> 3 of the group, which
  // holds logical 16-byte unit (l & 7) ^ (row & 7): the XOR order that keeps the fragment
  // reads (16 rows, one logical unit) bank-conflict free.
  const int grow = lane >> 3;
  const int unit = (lane & 7) ^ grow;
  const uint16_t* __restrict__ srca[kLoadsPerWave];
  const uint16_t* __restrict__ srcb[kLoadsPerWave];
  const uint16_t* __restrict__ wbase =
      reinterpret_cast<const uint16_t*>(op.w) + (long long)(routed ? e : 0) * op.estride;
#pragma unroll
  for (int i = 0; i < kLoadsPerWave; ++i) {
    const int row = (wave + 8 * i) * 8 + grow;  // 0..255
    long long wrow;
    if (MODE == kModeSwiglu) {
      const int g = rb * (PBN / 2) + (row >> 6) * 32 + (row & 31);  // gate row index
      wrow = (long long)g * op.ldw + (((row >> 5) & 1) ? op.up_off : 0);
    } else {
      wrow = (long long)min(rb * PBN + row, op.N - 1) * op.ldw;  // last block may be partial
    }
    srca[i] = wbase + wrow + unit * 8;
    const int r = min(r0 + row, r1 - 1);
    long long src;
    if (!routed)
      src = r - args.P;
    else if (op.in_map)
      src = args.order[r] / args.topk;
    else
      src = r;
    srcb[i] = op.in + src * op.ld_in + unit * 8;
  }
  char* lds = reinterpret_cast<char*>(smem);
  char* bring_lds = lds + kStagesA * kOpStage;
  auto issue_a = [&](int d) {
    char* st = lds + (d % kStagesA) * kOpStage;
#pragma unroll
    for (int i = 0; i < kLoadsPerWave; ++i)
      __builtin_amdgcn_global_load_lds(srca[i] + d * DKC, st + (wave + 8 * i) * 1024, 16, 0,
                                       kWeightCachePolicy);
  };
  // token-row groups past the tile's tokens are not loaded (their LDS rows keep stale data,
  // which only reaches MFMA output columns that are never stored): nb_loads of the wave's 4
  const int nb_loads = __builtin_amdgcn_readfirstlane(
      min(kLoadsPerWave, max(0, ((r1 - r0 + 7) / 8 - wave + 7) / 8)));
  auto issue_b = [&](int d) {
    char* st = bring_lds + (d % kStagesB) * kOpStage;
#pragma unroll
    for (int i = 0; i < kLoadsPerWave; ++i)
      if (i < nb_loads)
        __builtin_amdgcn_global_load_lds(srcb[i] + d * DKC, st + (wave + 8 * i) * 1024, 16, 0, 0);
  };
  // fragment read offsets of this lane (row lr of a 16-row block, logical unit s * 4 + kq)
  typedef __attribute__((address_space(3))) char lds_char;
  const uint32_t lds_base = (uint32_t)(uintptr_t)(lds_char*)lds;  // LDS byte address
  const uint32_t roff0 = (uint32_t)(lr * kRowBytes + ((kq ^ (lr & 7)) * 16));
  const uint32_t roff1 = (uint32_t)(lr * kRowBytes + (((4 + kq) ^ (lr & 7)) * 16));

  f32x4_t acc[4][8];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 8; ++b) acc[a][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int nblk = (ntok + 15) >> 4;
  const int nb = __builtin_amdgcn_readfirstlane(min(8, (nblk - wn + 1) >> 1));  // real blocks

  // Software pipeline over k-steps j (chunk d = j / 2, half s = j % 2): the fragments of
  // k-step j + 1 are read while k-step j is multiplied. At the first k-step of chunk d + 1
  // (after the barrier that makes it visible) the wave issues B(d + 2) then A(d + 3): weight
  // rows are requested three chunks before use, token rows two. The prologue issues A(0),
  // B(0), A(1), B(1), A(2) — the order the steps would have — so the loads younger than a
  // chunk's B load are exactly the next A load.
  const int nd = op.K / DKC;
  const int nk = 2 * nd;
  issue_a(0);
  if (nd > 0) issue_b(0);
  if (nd > 1) issue_a(1);
  if (nd > 1) issue_b(1);
  if (nd > 2) issue_a(2);
  Frags f0, f1;
  // younger than B(0): A(1), B(1), A(2)
  wait_loads(4 * (nd > 1) + nb_loads * (nd > 1) + 4 * (nd > 2));
  __builtin_amdgcn_s_barrier();
  read_frags(lds_base + roff0, lds_base + kStagesA * kOpStage + roff0, wm, wn, f0);
  frags_ready(f0);
  auto step = [&](int j, Frags& cur, Frags& nxt) {
    const bool more = j + 1 < nk;
    if (more) {
      const int jn = j + 1, dn = jn >> 1;
      if ((jn & 1) == 0) {
        // chunk dn: younger than B(dn) is A(dn + 1) if it was issued
        wait_loads(4 * (dn + 1 < nd));
        __builtin_amdgcn_s_barrier();
        if (dn + kAheadB < nd) issue_b(dn + kAheadB);
        if (dn + kAheadA < nd) issue_a(dn + kAheadA);
      }
      const uint32_t ro = (jn & 1) ? roff1 : roff0;
      read_frags(lds_base + (dn % kStagesA) * kOpStage + ro,
                 lds_base + (kStagesA + dn % kStagesB) * kOpStage + ro, wm, wn, nxt);
    }
    mma_frags(cur, nb, acc);
    if (more) frags_ready(nxt);
  };
  for (int j = 0; j < nk; j += 2) {
    step(j, f0, f1);
    step(j + 1, f1, f0);
  }

  // ---- epilogue: lane (q = kq, j = lr) holds rows 4q..4q+3 of token column j per block.
  const float* sc = op.scale ? op.scale + (long long)(routed ? e : 0) * op.sstride : nullptr;
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    if (b >= nb) break;
    const int rr = r0 + (2 * b + wn) * 16 + lr;
    if (rr >= r1) continue;
    const long long orow = routed ? (op.out_map ? args.order[rr] : rr) : rr - args.P;
    if (MODE == kModeSwiglu) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int n = rb * (PBN / 2) + wm * 32 + h * 16 + 4 * kq;
        float o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float g = acc[h][b][i], u = acc[2 + h][b][i];
          if (sc) {
            g *= sc[n + i];
            u *= sc[op.s_up_off + n + i];
          }
          g = rbf(g);
          u = rbf(u);
          o[i] = rbf(siluf_(g)) * u;
        }
        *reinterpret_cast<uint2*>(op.out + orow * op.ld_out + n) =
            make_uint2(pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3]));
      }
    } else {
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int n = rb * PBN + wm * 64 + a * 16 + 4 * kq;
        if (n >= op.N) break;  // N is a multiple of 16: n < N covers n + 3
        float o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = sc ? acc[a][b][i] * sc[n + i] : acc[a][b][i];
        *reinterpret_cast<uint2*>(op.out + orow * op.ld_out + n) =
            make_uint2(pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3]));
      }
    }
  }
}

// ---------------------------------------------------------------- fp8-e4m3 weights
//
// The same tile contract with e4m3 weight bytes (per-output-row fp32 scales on the fp32
// accumulator): a DMA chunk is 128 k, i.e. still 128 bytes of each weight row, so the weight
// stages keep the bf16 kernel's layout (256 rows x 128 B, XOR-swizzled 16-byte units) and
// their HBM access pattern while carrying twice the K. The token rows (bf16) of a 128-k
// chunk are 256 bytes each, so the token stages hold 128 tokens: a workgroup takes one
// half of a table tile (up to 256 sorted rows), the two halves of a tile being consecutive
// workgroups of one XCD, which stream the same weight rows together and share them in its
// L2. A fragment of the weights is 8 bytes of one row read from LDS and widened to bf16 in
// registers (exact), then v_mfma_f32_16x16x32_bf16 as in the bf16 kernel.
namespace {
constexpr int F8TOK = 128;                        // tokens per workgroup (half a table tile)
constexpr int F8KC = 128;                         // K elements per DMA chunk
constexpr int F8BRow = F8KC * 2;                  // token-row bytes per chunk: 256
}  // namespace

// Fragments of one double k-step (64 k) of a wave. The chunk's 128 k are read in a fixed
// permutation that both operands share (the products summed are the same): lane group kq
// of double step t takes weight unit 4 t + kq (16 e4m3 bytes, one conflict-free 16-byte LDS
// read) and uses its first 8 bytes in k-step 2 t, its last 8 in k-step 2 t + 1; the token
// fragments of those k-steps are the matching bf16 units 8 t + 2 kq and 8 t + 2 kq + 1.
struct Frags8 {
  u32x4v a[4];     // weight-row blocks, 16 e4m3 bytes each
  u32x4v b[2][4];  // [k-step][token block 2 b + wn]
};

// astage: the lane's weight offset for the double step; bstage0 / bstage1: its token
// offsets for the two k-steps.
__device__ __forceinline__ void read_frags8(uint32_t astage, uint32_t bstage0, uint32_t bstage1,
                                            Frags8& f) {
  f.a[0] = lds_read_frag<0 * 16 * kRowBytes>(astage);
  f.a[1] = lds_read_frag<1 * 16 * kRowBytes>(astage);
  f.a[2] = lds_read_frag<2 * 16 * kRowBytes>(astage);
  f.a[3] = lds_read_frag<3 * 16 * kRowBytes>(astage);
  f.b[0][0] = lds_read_frag<0 * 32 * F8BRow>(bstage0);
  f.b[0][1] = lds_read_frag<1 * 32 * F8BRow>(bstage0);
  f.b[0][2] = lds_read_frag<2 * 32 * F8BRow>(bstage0);
  f.b[0][3] = lds_read_frag<3 * 32 * F8BRow>(bstage0);
  f.b[1][0] = lds_read_frag<0 * 32 * F8BRow>(bstage1);
  f.b[1][1] = lds_read_frag<1 * 32 * F8BRow>(bstage1);
  f.b[1][2] = lds_read_frag<2 * 32 * F8BRow>(bstage1);
  f.b[1][3] = lds_read_frag<3 * 32 * F8BRow>(bstage1);
}
__device__ __forceinline__ void frags_ready8(Frags8& f) {
  lds_frags_ready();
#pragma unroll
  for (int a = 0; a < 4; ++a) after_wait(f.a[a]);
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int b = 0; b < 4; ++b) after_wait(f.b[h][b]);
}
// 8 e4m3 bytes -> bf16x8 (exact)
__device__ __forceinline__ u32x4v widen8(uint32_t lo, uint32_t hi) {
  u32x4v r;
  r.x = fp8x2_to_bf16x2<false>(lo);
  r.y = fp8x2_to_bf16x2<true>(lo);
  r.z = fp8x2_to_bf16x2<false>(hi);
  r.w = fp8x2_to_bf16x2<true>(hi);
  return r;
}
__device__ __forceinline__ void mma_frags8(const Frags8& f, int nb, f32x4_t (&acc)[4][4]) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    u32x4v a[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      a[i] = h ? widen8(f.a[i].z, f.a[i].w) : widen8(f.a[i].x, f.a[i].y);
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      if (b >= nb) break;
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i][b] = mfma_frag(a[i], f.b[h][b], acc[i][b]);
    }
  }
}

// One work item of the fp8 kernel: rows [r0, r1) (at most 128) of expert e against weight-row
// block rb: the whole DMA / MFMA pipeline of one tile and its epilogue.
template <int MODE>
__device__ __forceinline__ void f8_item(const GemmArgs& args, int e, int r0, int r1,
                                        int rb) {
  const bool routed = e < args.E;
  const GemmOperand& op = routed ? args.op[0] : args.op[1];
  constexpr int kOutPerWG = MODE == kModeSwiglu ? PBN / 2 : PBN;
  if (rb * kOutPerWG >= op.N) return;
  extern __shared__ uint4 smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 3;   // weight-row group (64 rows)
  const int wn = wave >> 2;  // token-block parity
  const int lr = lane & 15;
  const int kq = lane >> 4;
  const int ntok = r1 - r0;

  // ---- DMA sources. Weights: load i of the wave fills the 8-row group wave + 8 i of a
  // stage (128 bytes of each row), lane l physical unit l & 7 of row l >> 3, holding logical
  // unit (l & 7) ^ row. Token rows: load i fills the 4-row group wave + 8 i (256 bytes of
  // each row), lane l physical unit l & 15 of row l >> 4, holding logical unit
  // (l & 15) ^ (row & 15).
  const uint8_t* __restrict__ srca[kLoadsPerWave];
  const uint16_t* __restrict__ srcb[kLoadsPerWave];
  const uint8_t* __restrict__ wbase =
      reinterpret_cast<const uint8_t*>(op.w) + (long long)(routed ? e : 0) * op.estride;
  {
    const int grow = lane >> 3;
    const int unit = (lane & 7) ^ grow;
#pragma unroll
    for (int i = 0; i < kLoadsPerWave; ++i) {
      const int row = (wave + 8 * i) * 8 + grow;  // 0..255
      long long wrow;
      if (MODE == kModeSwiglu) {
        const int g = rb * (PBN / 2) + (row >> 6) * 32 + (row & 31);
        wrow = (long long)g * op.ldw + (((row >> 5) & 1) ? op.up_off : 0);
      } else {
        wrow = (long long)min(rb * PBN + row, op.N - 1) * op.ldw;
      }
      srca[i] = wbase + wrow + unit * 16;
    }
  }
  {
    const int brow = lane >> 4;
#pragma unroll
    for (int i = 0; i < kLoadsPerWave; ++i) {
      const int row = (wave + 8 * i) * 4 + brow;  // 0..127
      const int unit = (lane & 15) ^ (row & 15);
      const int r = min(r0 + row, r1 - 1);
      long long src;
      if (!routed)
        src = r - args.P;
      else if (op.in_map)
        src = args.order[r] / args.topk;
      else
        src = r;
      srcb[i] = op.in + src * op.ld_in + unit * 8;
    }
  }
  char* lds = reinterpret_cast<char*>(smem);
  char* bring_lds = lds + kStagesA * kOpStage;
  auto issue_a = [&](int d) {
    char* st = lds + (d % kStagesA) * kOpStage;
#pragma unroll
    for (int i = 0; i < kLoadsPerWave; ++i)
      __builtin_amdgcn_global_load_lds(srca[i] + d * F8KC, st + (wave + 8 * i) * 1024, 16, 0,
                                       kWeightCachePolicy);
  };
  const int nb_loads = __builtin_amdgcn_readfirstlane(
      min(kLoadsPerWave, max(0, ((ntok + 3) / 4 - wave + 7) / 8)));
  auto issue_b = [&](int d) {
    char* st = bring_lds + (d % kStagesB) * kOpStage;
#pragma unroll
    for (int i = 0; i < kLoadsPerWave; ++i)
      if (i < nb_loads)
        __builtin_amdgcn_global_load_lds(srcb[i] + d * F8KC, st + (wave + 8 * i) * 1024, 16, 0, 0);
  };
  // fragment offsets of this lane at k-step s of a chunk: weights row lr of a 16-row block,
  // 8 bytes at k = 32 s + 8 kq (logical unit 2 s + kq / 2, half kq & 1); token row lr of a
  // 16-row block, 16 bytes at logical unit 4 s + kq
  typedef __attribute__((address_space(3))) char lds_char;
  const uint32_t lds_base = (uint32_t)(uintptr_t)(lds_char*)lds;
  uint32_t roa[2], rob[2][2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    roa[t] = (uint32_t)(wm * 64 * kRowBytes + lr * kRowBytes + (((4 * t + kq) ^ (lr & 7)) * 16));
#pragma unroll
    for (int h = 0; h < 2; ++h)
      rob[t][h] = (uint32_t)(wn * 16 * F8BRow + lr * F8BRow + (((8 * t + 2 * kq + h) ^ lr) * 16));
  }

  f32x4_t acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int nblk = (ntok + 15) >> 4;
  const int nb = __builtin_amdgcn_readfirstlane(min(4, (nblk - wn + 1) >> 1));

  // Software pipeline as in the bf16 kernel, two double k-steps per chunk: at the first one
  // of chunk d + 1 the wave issues B(d + 2) then A(d + 3).
  const int nd = op.K / F8KC;
  const int nk = 2 * nd;
  issue_a(0);
  if (nd > 0) issue_b(0);
  if (nd > 1) issue_a(1);
  if (nd > 1) issue_b(1);
  if (nd > 2) issue_a(2);
  // the epilogue's row scales, requested now so that they arrive under the K loop
  const float* sc = op.scale ? op.scale + (long long)(routed ? e : 0) * op.sstride : nullptr;
  float scl[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int n;
      if (MODE == kModeSwiglu)  // blocks 0-1 gate rows, 2-3 the matching up rows
        n = rb * (PBN / 2) + wm * 32 + (a & 1) * 16 + 4 * kq + i + ((a >> 1) ? (int)op.s_up_off : 0);
      else
        n = min(rb * PBN + wm * 64 + a * 16 + 4 * kq + i, op.N - 1);
      scl[a][i] = sc ? sc[n] : 1.f;
    }
  Frags8 f0, f1;
  wait_loads(4 * (nd > 1) + nb_loads * (nd > 1) + 4 * (nd > 2));
  __builtin_amdgcn_s_barrier();
  read_frags8(lds_base + roa[0], lds_base + kStagesA * kOpStage + rob[0][0],
              lds_base + kStagesA * kOpStage + rob[0][1], f0);
  frags_ready8(f0);
  auto step = [&](int jj, Frags8& cur, Frags8& nxt) {
    const bool more = jj + 1 < nk;
    if (more) {
      const int jn = jj + 1, dn = jn >> 1, tn = jn & 1;
      if (tn == 0) {
        wait_loads(4 * (dn + 1 < nd));
        __builtin_amdgcn_s_barrier();
        if (dn + kAheadB < nd) issue_b(dn + kAheadB);
        if (dn + kAheadA < nd) issue_a(dn + kAheadA);
      }
      const uint32_t bst = lds_base + (kStagesA + dn % kStagesB) * kOpStage;
      read_frags8(lds_base + (dn % kStagesA) * kOpStage + roa[tn], bst + rob[tn][0],
                  bst + rob[tn][1], nxt);
    }
    mma_frags8(cur, nb, acc);
    if (more) frags_ready8(nxt);
  };
  for (int jj = 0; jj < nk; jj += 2) {
    step(jj, f0, f1);
    step(jj + 1, f1, f0);
  }

  // ---- epilogue: lane (q = kq, j = lr) holds rows 4q..4q+3 of token column j per block.
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    if (b >= nb) break;
    const int rr = r0 + (2 * b + wn) * 16 + lr;
    if (rr >= r1) continue;
    const long long orow = routed ? (op.out_map ? args.order[rr] : rr) : rr - args.P;
    if (MODE == kModeSwiglu) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int n = rb * (PBN / 2) + wm * 32 + h * 16 + 4 * kq;
        float o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float g = acc[h][b][i] * scl[h][i], u = acc[2 + h][b][i] * scl[2 + h][i];
          g = rbf(g);
          u = rbf(u);
          o[i] = rbf(siluf_(g)) * u;
        }
        *reinterpret_cast<uint2*>(op.out + orow * op.ld_out + n) =
            make_uint2(pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3]));
      }
    } else {
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int n = rb * PBN + wm * 64 + a * 16 + 4 * kq;
        if (n >= op.N) break;
        float o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = acc[a][b][i] * scl[a][i];
        *reinterpret_cast<uint2*>(op.out + orow * op.ld_out + n) =
            make_uint2(pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3]));
      }
    }
  }
}

// Persistent: one workgroup per CU (the LDS allows no more), each taking work items (tile,
// row block, token half) in a fixed order until the table's tiles are done. Short items
// (4 DMA chunks for the down projection) and the many empty halves would otherwise each
// pay a workgroup dispatch. Item order: round r of the grid covers 4 S (tile, row block)
// pairs p (S = workgroups per XCD); the two halves of a pair go to workgroups 8 apart, i.e.
// to one XCD at the same time, where they share the weight rows in its L2.
template <int MODE>
__global__ __launch_bounds__(kThreads, 1) void k_prefill_gemm_f8(GemmArgs args) {
  const int nrb = args.nrb;
  const int xcd = blockIdx.x & (kXcds - 1);
  const int slot = blockIdx.x / kXcds;
  const int S = gridDim.x / kXcds;
  const int half = slot & 1;
  const int npairs = args.MTgrid * nrb;
  const int ntiles = args.table ? args.table[3 * args.MT] : args.MTgrid;
  for (int p = (slot >> 1) * kXcds + xcd; p < npairs; p += 4 * S) {
    int tile = p / nrb;
    const int rb = p - tile * nrb;
    if (tile >= ntiles) break;  // the remaining items are past the table's tiles too
    int e, r0, r1;
    if (args.table) {
      if (args.shared_first > 0) {
        const int ns = min(args.shared_first, ntiles);
        tile = tile < ns ? ntiles - ns + tile : tile - ns;
      }
      e = args.table[tile];
      r0 = args.table[args.MT + tile];
      r1 = min(args.table[2 * args.MT + tile], r0 + PBM);
    } else {
      e = args.E;
      r0 = args.P + tile * PBM;
      if (r0 >= args.P + args.T) break;
      r1 = min(r0 + PBM, args.P + args.T);
    }
    r0 += half * F8TOK;
    r1 = min(r1, r0 + F8TOK);
    if (r0 >= r1) continue;
    f8_item<MODE>(args, e, r0, r1, rb);
    // the next item's loads refill the LDS stages: every wave is done with this item's
    // (its epilogue stores drained too, so the next item's vmcnt waits count its own loads)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }
}

int prefill_tile_rows() { return PBM; }

bool prefill_fits(int mode, const GemmOperand& op) {
  if (op.N <= 0) return true;
  // SWIGLU: whole 128-row gate/up blocks; PLAIN: any multiple of 16 rows (the last block of
  // 256 may be partial); K in whole chunks of the fp8 kernel
  const bool rows_ok = mode == kModeSwiglu ? op.N % (PBN / 2) == 0 : op.N % 16 == 0;
  return rows_ok && (op.fp8 ? op.K % F8KC == 0 : op.K % PKC == 0);
}

namespace {
// The kernels' dynamic LDS above the default limit, allowed once per device and mode.
hipError_t allow_lds(const void* fn, int mode, int bytes) {
  static std::mutex mu;
  static uint64_t done[4] = {0, 0, 0, 0};  // [kernel], bit d: device d
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return err;
  if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mu);
  if (done[mode] >> dev & 1) return hipSuccess;
  err = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (err == hipSuccess) done[mode] |= uint64_t(1) << dev;
  return err;
}
}  // namespace

hipError_t launch_prefill_gemm(int mode, const GemmArgs& a_in, int max_tiles, hipStream_t st) {
  GemmArgs a = a_in;
  if (!prefill_fits(mode, a.op[0]) || !prefill_fits(mode, a.op[1])) return hipErrorInvalidValue;
  const bool has0 = a.op[0].N > 0, has1 = a.op[1].N > 0;
  if (has0 && has1 && a.op[0].fp8 != a.op[1].fp8) {
    // one weight type per kernel: the routed tiles, then the shared expert's (the table's
    // routed tiles exit at once in the second launch)
    GemmArgs r = a, v = a;
    r.op[1].N = 0;
    v.op[0].N = 0;
    hipError_t err = launch_prefill_gemm(mode, r, max_tiles, st);
    return err != hipSuccess ? err : launch_prefill_gemm(mode, v, max_tiles, st);
  }
  const bool f8 = (has0 && a.op[0].fp8) || (has1 && a.op[1].fp8);
  const int out_per_wg = mode == kModeSwiglu ? PBN / 2 : PBN;
  const int nmax = a.op[0].N > a.op[1].N ? a.op[0].N : a.op[1].N;
  a.nrb = (nmax + out_per_wg - 1) / out_per_wg;
  if (a.nrb <= 0 || max_tiles <= 0) return hipSuccess;
  const size_t lds = (size_t)kLdsBytes;
  a.MTgrid = max_tiles;
  a.shared_first = 0;
  if (a.table && a.op[0].N > 0 && a.op[1].N > 0) {
    const char* env = knob(kKnobPrefillSharedFirst);
    if (!(env && env[0] == '0')) a.shared_first = (a.T + PBM - 1) / PBM;
  }
  long long grid = (long long)((max_tiles + kXcds - 1) / kXcds) * kXcds * a.nrb;
  if (f8) {
    // persistent: one workgroup per CU, a whole number of pairs of workgroups per XCD
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return hipErrorInvalidDevice;
    grid = (long long)((cus + 2 * kXcds - 1) / (2 * kXcds)) * 2 * kXcds;
  }
  if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
  const void* fn = mode == kModeSwiglu
                       ? (f8 ? reinterpret_cast<const void*>(&k_prefill_gemm_f8<kModeSwiglu>)
                             : reinterpret_cast<const void*>(&k_prefill_gemm<kModeSwiglu>))
                       : (f8 ? reinterpret_cast<const void*>(&k_prefill_gemm_f8<kModePlain>)
                             : reinterpret_cast<const void*>(&k_prefill_gemm<kModePlain>));
  hipError_t err = allow_lds(fn, mode + (f8 ? 2 : 0), (int)lds);
  if (err != hipSuccess) return err;
  if (f8) {
    if (mode == kModeSwiglu)
      hipLaunchKernelGGL(k_prefill_gemm_f8<kModeSwiglu>, dim3((unsigned)grid), dim3(kThreads), lds, st, a);
    else
      hipLaunchKernelGGL(k_prefill_gemm_f8<kModePlain>, dim3((unsigned)grid), dim3(kThreads), lds, st, a);
    return hipGetLastError();
  }
  if (mode == kModeSwiglu)
    hipLaunchKernelGGL(k_prefill_gemm<kModeSwiglu>, dim3((unsigned)grid), dim3(kThreads), lds, st, a);
  else
    hipLaunchKernelGGL(k_prefill_gemm<kModePlain>, dim3((unsigned)grid), dim3(kThreads), lds, st, a);
  return hipGetLastError();
}

}  // namespace moe
