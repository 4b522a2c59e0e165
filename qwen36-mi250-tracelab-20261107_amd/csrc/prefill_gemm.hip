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
// The same tiles (256 weight rows x up to 256 sorted rows) with e4m3 weight bytes and
// per-output-row fp32 scales on the fp32 accumulator. A DMA chunk is 64 k as in the bf16
// kernel, so the token-row stages are the bf16 kernel's (256 rows x 128 bytes), while a
// weight stage is 256 rows x 64 bytes (16 KiB): the ring holds five of them (four chunks
// requested ahead, 144 KiB of LDS in all). A weight DMA load of a wave fills 16 rows x 64
// bytes; lane l writes physical 16-byte unit l & 3 of row l >> 2 of its group, holding
// logical unit (l & 3) ^ ((row >> 1) & 3), which keeps the fragment reads (8 rows of one
// 16-byte read group) conflict-free.
//
// The weight loads use the default cache policy: unlike the bf16 kernel's, the non-temporal
// one measured slower here (grouped gate_up / down at 4096 tokens 261 / 189 against 248 /
// 181 µs). A deeper or shallower weight ring (6 or 4 stages) changed little.
//
// The chunk's k order is permuted the same way in both operands (the same products are
// summed): lane group kq reads weight unit kq (16 e4m3 bytes, one ds_read_b128) once per
// chunk and feeds its first 8 bytes to the chunk's k-step 0 and its last 8 to k-step 1,
// against token units 2 kq and 2 kq + 1. The weights are widened to bf16 in registers
// (gfx950's scaled conversion, scale 1: exact) just before their MFMAs.
namespace {
constexpr int F8RowBytes = DKC;                   // weight bytes of a row per chunk: 64
constexpr int F8Stage = 256 * F8RowBytes;         // 16 KiB
constexpr int F8StagesA = 5, F8AheadA = 4;
constexpr int F8ALoads = 256 / 16 / 8;            // weight DMA loads per wave per chunk: 2
constexpr int F8LdsBytes = F8StagesA * F8Stage + kStagesB * kOpStage;  // 144 KiB
static_assert(F8AheadA == F8StagesA - 1, "weight ring: chunk d + S - 1 into chunk d - 1's stage");
}  // namespace

// 8 e4m3 bytes -> bf16x8 (exact)
__device__ __forceinline__ u32x4v widen8(uint32_t lo, uint32_t hi) {
  u32x4v r;
  r.x = fp8x2_to_bf16x2<false>(lo);
  r.y = fp8x2_to_bf16x2<true>(lo);
  r.z = fp8x2_to_bf16x2<false>(hi);
  r.w = fp8x2_to_bf16x2<true>(hi);
  return r;
}
// Token fragments of one k-step (the wave's 8 blocks 2 b + wn) from the B stage at bstage.
__device__ __forceinline__ void read_bfrags(uint32_t bstage, u32x4v (&b)[8]) {
  b[0] = lds_read_frag<0 * kBlkBytes>(bstage);
  b[1] = lds_read_frag<2 * kBlkBytes>(bstage);
  b[2] = lds_read_frag<4 * kBlkBytes>(bstage);
  b[3] = lds_read_frag<6 * kBlkBytes>(bstage);
  b[4] = lds_read_frag<8 * kBlkBytes>(bstage);
  b[5] = lds_read_frag<10 * kBlkBytes>(bstage);
  b[6] = lds_read_frag<12 * kBlkBytes>(bstage);
  b[7] = lds_read_frag<14 * kBlkBytes>(bstage);
}
// Weight fragments of one chunk (4 row blocks of 16 rows, 16 bytes per lane).
__device__ __forceinline__ void read_afrags8(uint32_t astage, u32x4v (&a)[4]) {
  a[0] = lds_read_frag<0 * 16 * F8RowBytes>(astage);
  a[1] = lds_read_frag<1 * 16 * F8RowBytes>(astage);
  a[2] = lds_read_frag<2 * 16 * F8RowBytes>(astage);
  a[3] = lds_read_frag<3 * 16 * F8RowBytes>(astage);
}
template <int N>
__device__ __forceinline__ void tie(u32x4v (&v)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) after_wait(v[i]);
}
// k-step h of a chunk: weight halves h of a[], token fragments b[], first nb blocks.
__device__ __forceinline__ void mma8(const u32x4v (&a)[4], int h, const u32x4v (&b)[8], int nb,
                                     f32x4_t (&acc)[4][8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const u32x4v w = h ? widen8(a[i].z, a[i].w) : widen8(a[i].x, a[i].y);
#pragma unroll
    for (int bb = 0; bb < 8; ++bb) {
      if (bb >= nb) break;
      acc[i][bb] = mfma_frag(w, b[bb], acc[i][bb]);
    }
  }
}

template <int MODE>
__global__ __launch_bounds__(kThreads, 1) void k_prefill_gemm_f8(GemmArgs args) {
  extern __shared__ uint4 smem[];  // A ring [F8StagesA][16 KiB], B ring [kStagesB][32 KiB]

  // tile / row-block order, table lookup and bounds: as k_prefill_gemm
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
      const int ns = min(args.shared_first, ntiles);
      tile = tile < ns ? ntiles - ns + tile : tile - ns;
    }
    e = args.table[tile];
    r0 = args.table[args.MT + tile];
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
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 3;   // weight-row group (64 rows)
  const int wn = wave >> 2;  // token-block parity
  const int lr = lane & 15;
  const int kq = lane >> 4;
  const int ntok = r1 - r0;

  // ---- DMA sources: weights (load i of the wave: 16-row group wave + 8 i), token rows (as
  // k_prefill_gemm: 8-row group wave + 8 i, 128 bytes of each row)
  const uint8_t* __restrict__ srca[F8ALoads];
  const uint16_t* __restrict__ srcb[kLoadsPerWave];
  {
    const uint8_t* __restrict__ wbase =
        reinterpret_cast<const uint8_t*>(op.w) + (long long)(routed ? e : 0) * op.estride;
    const int arow = lane >> 2;
#pragma unroll
    for (int i = 0; i < F8ALoads; ++i) {
      const int row = (wave + 8 * i) * 16 + arow;  // 0..255
      const int unit = (lane & 3) ^ ((row >> 1) & 3);
      long long wrow;
      if (MODE == kModeSwiglu) {
        const int g = rb * (PBN / 2) + (row >> 6) * 32 + (row & 31);
        wrow = (long long)g * op.ldw + (((row >> 5) & 1) ? op.up_off : 0);
      } else {
        wrow = (long long)min(rb * PBN + row, op.N - 1) * op.ldw;
      }
      srca[i] = wbase + wrow + unit * 16;
    }
    // token rows: physical unit q = (l & 7) ^ row holds logical unit 2 (q & 3) + (q >> 2), so
    // that the units 2 kq + h that k-step h reads sit where the bf16 kernel's k-step reads
    // them (physical (4 h + kq) ^ row): that pattern is conflict-free, 2 kq + h at the
    // physical unit was not (3.2 bank-conflict cycles per LDS instruction)
    const int grow = lane >> 3;
    const int bq = (lane & 7) ^ grow;
    const int bunit = 2 * (bq & 3) + (bq >> 2);
#pragma unroll
    for (int i = 0; i < kLoadsPerWave; ++i) {
      const int row = (wave + 8 * i) * 8 + grow;
      const int r = min(r0 + row, r1 - 1);
      long long src;
      if (!routed)
        src = r - args.P;
      else if (op.in_map)
        src = args.order[r] / args.topk;
      else
        src = r;
      srcb[i] = op.in + src * op.ld_in + bunit * 8;
    }
  }
  char* lds = reinterpret_cast<char*>(smem);
  char* bring_lds = lds + F8StagesA * F8Stage;
  auto issue_a = [&](int d) {
    char* st = lds + (d % F8StagesA) * F8Stage;
#pragma unroll
    for (int i = 0; i < F8ALoads; ++i)
      __builtin_amdgcn_global_load_lds(srca[i] + d * F8RowBytes, st + (wave + 8 * i) * 1024, 16,
                                       0, 0);
  };
  const int nb_loads = __builtin_amdgcn_readfirstlane(
      min(kLoadsPerWave, max(0, ((r1 - r0 + 7) / 8 - wave + 7) / 8)));
  auto issue_b = [&](int d) {
    char* st = bring_lds + (d % kStagesB) * kOpStage;
#pragma unroll
    for (int i = 0; i < kLoadsPerWave; ++i)
      if (i < nb_loads)
        __builtin_amdgcn_global_load_lds(srcb[i] + d * DKC, st + (wave + 8 * i) * 1024, 16, 0, 0);
  };
  typedef __attribute__((address_space(3))) char lds_char;
  const uint32_t lds_base = (uint32_t)(uintptr_t)(lds_char*)lds;
  // weight fragment: row lr of a 16-row block, logical unit kq; token fragment of k-step h:
  // row lr, logical unit 2 kq + h (stored at physical (4 h + kq) ^ row)
  const uint32_t ra = (uint32_t)(wm * 64 * F8RowBytes + lr * F8RowBytes +
                                 ((kq ^ ((lr >> 1) & 3)) * 16));
  const uint32_t rbo0 = (uint32_t)(wn * kBlkBytes + lr * kRowBytes + ((kq ^ (lr & 7)) * 16));
  const uint32_t rbo1 = (uint32_t)(wn * kBlkBytes + lr * kRowBytes + (((4 + kq) ^ (lr & 7)) * 16));

  f32x4_t acc[4][8];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 8; ++b) acc[a][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int nblk = (ntok + 15) >> 4;
  const int nb = __builtin_amdgcn_readfirstlane(min(8, (nblk - wn + 1) >> 1));

  // Pipeline: chunk d's weight fragments are read at its k-step 0 and kept for k-step 1;
  // the token fragments of each k-step are read while the previous one is multiplied. Load
  // order: A(0 .. S - 3), B(0), A(S - 2), B(1), A(S - 1), then at chunk d + 1's first k-step
  // B(d + 2), A(d + S), so that the loads younger than B(d) are exactly A(d + S - 2).
  const int nd = op.K / DKC;
  const int nk = 2 * nd;
  for (int d = 0; d < F8AheadA - 1; ++d)
    if (d < nd) issue_a(d);
  if (nd > 0) issue_b(0);
  if (F8AheadA - 1 < nd) issue_a(F8AheadA - 1);
  if (nd > 1) issue_b(1);
  if (F8AheadA < nd) issue_a(F8AheadA);
  // younger than B(0): A(S - 2), B(1), A(S - 1)
  wait_loads(F8ALoads * (F8AheadA - 1 < nd) + nb_loads * (nd > 1) + F8ALoads * (F8AheadA < nd));
  __builtin_amdgcn_s_barrier();
  u32x4v acur[4], anxt[4], b0[8], b1[8];
  read_afrags8(lds_base + ra, acur);
  read_bfrags(lds_base + F8StagesA * F8Stage + rbo0, b0);
  lds_frags_ready();
  tie(acur);
  tie(b0);
  for (int d = 0; d < nd; ++d) {
    const uint32_t bst = lds_base + F8StagesA * F8Stage + (d % kStagesB) * kOpStage;
    // k-step 0 of chunk d (weights acur, tokens b0) while k-step 1's tokens are read
    read_bfrags(bst + rbo1, b1);
    mma8(acur, 0, b0, nb, acc);
    lds_frags_ready();
    tie(b1);
    // k-step 1 while chunk d + 1's weights and k-step-0 tokens are read
    const bool more = d + 1 < nd;
    if (more) {
      wait_loads(F8ALoads * (d + F8AheadA < nd));
      __builtin_amdgcn_s_barrier();
      if (d + 2 < nd) issue_b(d + 2);
      if (d + 1 + F8AheadA < nd) issue_a(d + 1 + F8AheadA);
      read_afrags8(lds_base + ((d + 1) % F8StagesA) * F8Stage + ra, anxt);
      read_bfrags(lds_base + F8StagesA * F8Stage + ((d + 1) % kStagesB) * kOpStage + rbo0, b0);
    }
    mma8(acur, 1, b1, nb, acc);
    if (more) {
      lds_frags_ready();
      tie(anxt);
      tie(b0);
#pragma unroll
      for (int i = 0; i < 4; ++i) acur[i] = anxt[i];
    }
  }

  // ---- epilogue (k_prefill_gemm's), the row scales requested together first
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
          float g = rbf(acc[h][b][i] * scl[h][i]);
          float u = rbf(acc[2 + h][b][i] * scl[2 + h][i]);
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

int prefill_tile_rows() { return PBM; }

bool prefill_fits(int mode, const GemmOperand& op) {
  if (op.N <= 0) return true;
  // SWIGLU: whole 128-row gate/up blocks; PLAIN: any multiple of 16 rows (the last block of
  // 256 may be partial); K in whole chunks of the fp8 kernel
  const bool rows_ok = mode == kModeSwiglu ? op.N % (PBN / 2) == 0 : op.N % 16 == 0;
  return rows_ok && (op.fp8 ? op.K % DKC == 0 : op.K % PKC == 0);
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
  const long long grid = (long long)((max_tiles + kXcds - 1) / kXcds) * kXcds * a.nrb;
  if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
  const size_t lds_k = f8 ? (size_t)F8LdsBytes : lds;
  const void* fn = mode == kModeSwiglu
                       ? (f8 ? reinterpret_cast<const void*>(&k_prefill_gemm_f8<kModeSwiglu>)
                             : reinterpret_cast<const void*>(&k_prefill_gemm<kModeSwiglu>))
                       : (f8 ? reinterpret_cast<const void*>(&k_prefill_gemm_f8<kModePlain>)
                             : reinterpret_cast<const void*>(&k_prefill_gemm<kModePlain>));
  hipError_t err = allow_lds(fn, mode + (f8 ? 2 : 0), (int)lds_k);
  if (err != hipSuccess) return err;
  if (f8) {
    if (mode == kModeSwiglu)
      hipLaunchKernelGGL(k_prefill_gemm_f8<kModeSwiglu>, dim3((unsigned)grid), dim3(kThreads), lds_k, st, a);
    else
      hipLaunchKernelGGL(k_prefill_gemm_f8<kModePlain>, dim3((unsigned)grid), dim3(kThreads), lds_k, st, a);
    return hipGetLastError();
  }
  if (mode == kModeSwiglu)
    hipLaunchKernelGGL(k_prefill_gemm<kModeSwiglu>, dim3((unsigned)grid), dim3(kThreads), lds, st, a);
  else
    hipLaunchKernelGGL(k_prefill_gemm<kModePlain>, dim3((unsigned)grid), dim3(kThreads), lds, st, a);
  return hipGetLastError();
}

}  // namespace moe
