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
// Pipeline. K runs in chunks of 32 (one MFMA k-step). A chunk of both operands (256 + 256
// rows x 64 B) is 32 blocks of 16 rows x 64 B; each block is one 1 KiB global -> LDS DMA
// load of a wave (global_load_lds_dwordx4: no registers on the way), and an MFMA fragment
// is one 1 KiB LDS read of a block. Inside a block the four 16-byte units of row r sit in
// the order u ^ ((r >> 2) & 3), which makes the fragment reads bank-conflict free. Four LDS
// stages: while chunk c is multiplied, the fragments of chunk c + 1 are being read into
// registers and the DMA loads of chunks c + 2 and c + 3 are in flight.
// The fragment reads are issued by inline asm with explicit lgkmcnt waits and the stages are
// fenced by explicit vmcnt waits, because the compiler's own waits would drain every
// outstanding DMA load before each LDS read.
#include <stdlib.h>

#include "moe_common.h"
#include "expert_gemm.h"

#ifndef MOE_PF_TRACE
#define MOE_PF_TRACE(tag, c)  // timing hook of the kernel's own benchmarks; no-op here
#endif

namespace moe {

namespace {
constexpr int PBM = 256;                          // tokens per tile
constexpr int PBN = 256;                          // weight rows per workgroup
constexpr int PKC = 32;                           // K elements per chunk
constexpr int kBlkBytes = 1024;                   // 16 rows x 32 k x 2 B
constexpr int kBlocks = (PBN + PBM) / 16;         // blocks per stage (A then B)
constexpr int kStageBytes = kBlocks * kBlkBytes;  // 32 KiB
constexpr int kStages = 5;
constexpr int kThreads = 512;
constexpr int kXcds = 8;                          // XCDs of an MI355X (round-robin dispatch)
constexpr int kWaves = kThreads / 64;
constexpr int kLoadsPerWave = kBlocks / kWaves;   // DMA loads per wave per chunk (4)
static_assert(kLoadsPerWave == 4, "vmcnt accounting below assumes 4 loads per chunk");
static_assert(kStages <= 5, "wait_chunks covers up to three younger chunks");
}  // namespace

typedef unsigned u32x4v __attribute__((ext_vector_type(4)));

template <int OFF>
__device__ __forceinline__ u32x4v lds_read_frag(uint32_t addr) {
  u32x4v r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}
__device__ __forceinline__ void lds_frags_ready() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}
// Ties a fragment to the wait above: its users cannot move before it.
__device__ __forceinline__ void after_wait(u32x4v& v) { asm volatile("" : "+v"(v)); }

__device__ __forceinline__ f32x4_t mfma_frag(u32x4v a, u32x4v b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// MFMA fragments of one chunk for a wave: 4 weight-row blocks, 8 token blocks.
struct Frags {
  u32x4v a[4], b[8];
};

// Issue the wave's 12 fragment reads of the stage at `base` (+ this lane's unit offset);
// they complete at frags_ready.
__device__ __forceinline__ void read_frags(uint32_t base, int wm, int wn, Frags& f) {
  const uint32_t abase = base + wm * 4 * kBlkBytes;
  const uint32_t bbase = base + (16 + wn) * kBlkBytes;
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

// Wait until at most `younger` chunks of this wave's DMA loads are still in flight.
__device__ __forceinline__ void wait_chunks(int younger) {
  if (younger >= 3)
    asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
  else if (younger == 2)
    asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  else if (younger == 1)
    asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
  else
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

template <int MODE>
__global__ __launch_bounds__(kThreads, 1) void k_prefill_gemm(GemmArgs args) {
  extern __shared__ uint4 smem[];  // [kStages][kBlocks][1 KiB]

  // XCD-aware order: workgroup b runs on XCD b % 8, so the nrb workgroups of one tile get
  // ids 8 apart (same XCD, dispatched together) and share the tile's token rows in that
  // XCD's L2 instead of fetching them once per XCD.
  const int nrb = args.nrb;
  const int xcd = blockIdx.x & (kXcds - 1);
  const int j = blockIdx.x / kXcds;
  const int tile = (j / nrb) * kXcds + xcd;
  const int rb = j - (j / nrb) * nrb;
  if (tile >= args.MTgrid) return;
  int e, r0, r1;
  if (args.table) {
    if (tile >= args.table[3 * args.MT]) return;
    e = args.table[tile];
    r0 = args.table[args.MT + tile];
    r1 = args.table[2 * args.MT + tile];
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
  const int nch = op.K / PKC;
  const int ntok = r1 - r0;

  // ---- DMA sources: this wave loads blocks wave + 8 i (i < 4) of every stage: A blocks
  // wave, wave + 8 and B blocks wave, wave + 8. Lane l fills unit l & 3 of row l >> 2 of the
  // block, i.e. logical 16-byte unit (l & 3) ^ ((row >> 2) & 3) of that row.
  const int brow = lane >> 2;
  const int unit = (lane & 3) ^ ((brow >> 2) & 3);
  const uint16_t* __restrict__ src[kLoadsPerWave];
  const uint16_t* __restrict__ wbase =
      reinterpret_cast<const uint16_t*>(op.w) + (long long)(routed ? e : 0) * op.estride;
#pragma unroll
  for (int i = 0; i < kLoadsPerWave; ++i) {
    const int blk = wave + 8 * i;  // 0..31
    if (blk < 16) {
      const int row = blk * 16 + brow;
      long long wrow;
      if (MODE == kModeSwiglu) {
        const int g = rb * (PBN / 2) + (row >> 6) * 32 + (row & 31);  // gate row index
        wrow = (long long)g * op.ldw + (((row >> 5) & 1) ? op.up_off : 0);
      } else {
        wrow = (long long)min(rb * PBN + row, op.N - 1) * op.ldw;  // last block may be partial
      }
      src[i] = wbase + wrow + unit * 8;
    } else {
      const int t = (blk - 16) * 16 + brow;
      const int r = min(r0 + t, r1 - 1);
      long long s;
      if (!routed)
        s = r - args.P;
      else if (op.in_map)
        s = args.order[r] / args.topk;
      else
        s = r;
      src[i] = op.in + s * op.ld_in + unit * 8;
    }
  }
  char* lds = reinterpret_cast<char*>(smem);
  auto issue = [&](int c) {
    char* st = lds + (c % kStages) * kStageBytes;
#pragma unroll
    for (int i = 0; i < kLoadsPerWave; ++i)
      __builtin_amdgcn_global_load_lds(src[i] + c * PKC, st + (wave + 8 * i) * kBlkBytes, 16, 0, 0);
  };
  // fragment read offset of this lane inside a block: row lr, logical unit kq
  const uint32_t roff = (uint32_t)(lr * 64 + ((kq ^ ((lr >> 2) & 3)) * 16));
  typedef __attribute__((address_space(3))) char lds_char;
  const uint32_t lds_base = (uint32_t)(uintptr_t)(lds_char*)lds;  // LDS byte address

  f32x4_t acc[4][8];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 8; ++b) acc[a][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int nblk = (ntok + 15) >> 4;
  const int nb = __builtin_amdgcn_readfirstlane(min(8, (nblk - wn + 1) >> 1));  // real blocks

  // Software pipeline: the fragments of chunk c + 1 are read from LDS while chunk c is
  // multiplied; DMA loads run kStages - 2 chunks ahead of the fragment reads.
  for (int c = 0; c < kStages - 1 && c < nch; ++c) issue(c);
  Frags f0, f1;
  wait_chunks(min(kStages - 2, nch - 1));
  __builtin_amdgcn_s_barrier();
  read_frags(lds_base + roff, wm, wn, f0);
  frags_ready(f0);
  auto step = [&](int c, Frags& cur, Frags& nxt) {
    const bool more = c + 1 < nch;
    MOE_PF_TRACE(0, c);
    if (more) {
      wait_chunks(min(kStages - 3, nch - 2 - c));
      MOE_PF_TRACE(1, c);
      __builtin_amdgcn_s_barrier();
      MOE_PF_TRACE(2, c);
      if (c + kStages - 1 < nch) issue(c + kStages - 1);
      read_frags(lds_base + ((c + 1) % kStages) * kStageBytes + roff, wm, wn, nxt);
    }
    mma_frags(cur, nb, acc);
    MOE_PF_TRACE(3, c);
    if (more) frags_ready(nxt);
    MOE_PF_TRACE(4, c);
  };
  for (int c = 0; c < nch; c += 2) {
    step(c, f0, f1);
    if (c + 1 < nch) step(c + 1, f1, f0);
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

int prefill_tile_rows() { return PBM; }

bool prefill_fits(int mode, const GemmOperand& op) {
  if (op.N <= 0) return true;
  // SWIGLU: whole 128-row gate/up blocks; PLAIN: any multiple of 16 rows (the last block of
  // 256 may be partial)
  const bool rows_ok = mode == kModeSwiglu ? op.N % (PBN / 2) == 0 : op.N % 16 == 0;
  return !op.fp8 && rows_ok && op.K % PKC == 0;
}

hipError_t launch_prefill_gemm(int mode, const GemmArgs& a_in, int max_tiles, hipStream_t st) {
  GemmArgs a = a_in;
  if (!prefill_fits(mode, a.op[0]) || !prefill_fits(mode, a.op[1])) return hipErrorInvalidValue;
  if (const char* env = getenv("MOE_PREFILL_DEBUG")) a.dbg = atoi(env);  // timing experiments
  const int out_per_wg = mode == kModeSwiglu ? PBN / 2 : PBN;
  const int nmax = a.op[0].N > a.op[1].N ? a.op[0].N : a.op[1].N;
  a.nrb = (nmax + out_per_wg - 1) / out_per_wg;
  if (a.nrb <= 0 || max_tiles <= 0) return hipSuccess;
  const size_t lds = (size_t)kStages * kStageBytes;
  a.MTgrid = max_tiles;
  const long long grid = (long long)((max_tiles + kXcds - 1) / kXcds) * kXcds * a.nrb;
  if (mode == kModeSwiglu) {
    static bool attr = false;
    if (!attr) {
      hipFuncSetAttribute(reinterpret_cast<const void*>(&k_prefill_gemm<kModeSwiglu>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      attr = true;
    }
    hipLaunchKernelGGL(k_prefill_gemm<kModeSwiglu>, dim3((unsigned)grid), dim3(kThreads), lds, st, a);
  } else {
    static bool attr = false;
    if (!attr) {
      hipFuncSetAttribute(reinterpret_cast<const void*>(&k_prefill_gemm<kModePlain>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      attr = true;
    }
    hipLaunchKernelGGL(k_prefill_gemm<kModePlain>, dim3((unsigned)grid), dim3(kThreads), lds, st, a);
  }
  return hipGetLastError();
}

}  // namespace moe
