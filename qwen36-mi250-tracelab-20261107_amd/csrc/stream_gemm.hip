// Expert-grouped, weight-streaming MFMA GEMM for gfx950 (subsystems a1, a4, a5, a6, a12).
//
// One kernel serves the decode-side projections of the MoE block:
//   * router logits        out[t, n]  = bf16(x_t . Wr[n])                 (PLAIN)
//   * expert gate_up       act[r, n]  = bf16(bf16(silu(bf16 g)) * bf16 u)  (SWIGLU)
//                          g = x_tok(r) . Wg[e, n], u = x_tok(r) . Wu[e, n]
//   * expert down          y[pair(r), n] = bf16(act[r] . Wd[e, n])          (PLAIN)
// The rounding points are those of Transformers' batched_mm experts path
// (transformers/integrations/moe.py:112-176) and of engine/fast/kernels.py:88-164.
//
// Work decomposition. The sort kernel groups the (token, expert) pairs by expert into
// tiles of up to BM = 16 * TOKB sorted rows of ONE expert (the tile table). A workgroup
// takes one tile and one block of weight rows; every weight element of the block is
// read from HBM exactly once per tile and multiplied against all of the tile's tokens
// (expert de-duplication across the batch). Weights stream straight from HBM into the
// MFMA A operand (16-byte loads, 64 contiguous bytes per row per load instruction); the
// token rows are the B operand (16 tokens per v_mfma_f32_16x16x32_bf16, from L2).
// A workgroup has WR x WK waves: WR blocks of 16 weight rows, each split WK ways along
// K; the K partial sums are reduced through LDS in a fixed order (deterministic).
// SWIGLU interleaves 8 gate rows and the matching 8 up rows in one 16-row MFMA tile so
// the epilogue pairs them in registers.
//
// fp8-e4m3 weights (per-output-row fp32 scales) are converted to bf16 in registers
// (exact) and the scale is applied to the fp32 accumulator before the bf16 rounding:
// sum_k s_n q_nk x_k = s_n sum_k q_nk x_k.
#include "moe_common.h"
#include "stream_gemm.h"

namespace moe {

// HAS_FP8: the launch may hold an fp8 operand; each operand's own ``fp8`` flag picks the
// bf16 or the fp8 main loop (a block's routed experts may be fp8 while its shared expert
// is bf16).
template <int MODE, int WR, int WK, int S, int TOKB, bool HAS_FP8>
__global__ __launch_bounds__(64 * WR * WK) void k_stream_gemm(GemmArgs args) {
  constexpr int kRowsPerWave = 16;
  constexpr int kOutRowsPerWG = (MODE == kModeSwiglu ? 8 : 16) * WR;
  constexpr int BM = 16 * TOKB;
  __shared__ f32x4_t red[(WK > 1 ? (WK - 1) : 1) * WR * TOKB * kWave];

  const int nrb = args.nrb;
  const int tile = blockIdx.x / nrb;
  const int rb = blockIdx.x - tile * nrb;

  int e, r0, r1;
  if (args.table) {
    if (tile >= args.table[3 * args.MT]) return;
    e = args.table[tile];
    r0 = args.table[args.MT + tile];
    r1 = args.table[2 * args.MT + tile];
  } else {
    e = args.E;
    r0 = args.P + tile * BM;
    if (r0 >= args.P + args.T) return;
    r1 = min(r0 + BM, args.P + args.T);
  }
  const bool routed = e < args.E;
  const GemmOperand& op = routed ? args.op[0] : args.op[1];
  if (rb * kOutRowsPerWG >= op.N) return;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wr = wave % WR;
  const int wk = wave / WR;
  const int lr = lane & 15;
  const int kq = lane >> 4;
  const int Kw = op.K / WK;
  const int kbeg = wk * Kw;

  // This lane's weight row (A operand row lr of the wave's 16-row tile).
  long long wrow_off;
  int obase;  // first output row (PLAIN) / gate row (SWIGLU) of the wave
  if (MODE == kModeSwiglu) {
    obase = rb * kOutRowsPerWG + wr * 8;
    wrow_off = (long long)(obase + (lr & 7)) * op.ldw + (lr >= 8 ? op.up_off : 0);
  } else {
    obase = rb * kOutRowsPerWG + wr * kRowsPerWave;
    wrow_off = (long long)(obase + lr) * op.ldw;
  }
  wrow_off += (long long)(routed ? e : 0) * op.estride + kbeg;

  // Token rows: tile rows r0 + tb*16 + lr (clamped; the padded columns are discarded).
  const int ntb = (r1 - r0 + 15) >> 4;
  long long brow[TOKB];
#pragma unroll
  for (int tb = 0; tb < TOKB; ++tb) {
    int rr = min(r0 + tb * 16 + lr, r1 - 1);
    int src;
    if (!routed)
      src = rr - args.P;
    else if (op.in_map)
      src = args.order[rr] / args.topk;
    else
      src = rr;
    brow[tb] = (long long)src * op.ld_in + kbeg;
  }

  f32x4_t acc[TOKB];
#pragma unroll
  for (int tb = 0; tb < TOKB; ++tb) acc[tb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const uint16_t* __restrict__ xin = op.in;
  if (!HAS_FP8 || !op.fp8) {
    constexpr int kChunk = 32 * S;  // K elements per iteration
    const uint16_t* __restrict__ wp = reinterpret_cast<const uint16_t*>(op.w) + wrow_off + kq * 8;
    for (int kc = 0; kc < Kw; kc += kChunk) {
      uint4 a[S];
#pragma unroll
      for (int s = 0; s < S; ++s) a[s] = ld16(wp + kc + s * 32);
#pragma unroll
      for (int tb = 0; tb < TOKB; ++tb) {
        if (tb < ntb) {
          const uint16_t* xp = xin + brow[tb] + kq * 8 + kc;
          uint4 b[S];
#pragma unroll
          for (int s = 0; s < S; ++s) b[s] = ld16(xp + s * 32);
#pragma unroll
          for (int s = 0; s < S; ++s) acc[tb] = mfma16x16x32(a[s], b[s], acc[tb]);
        }
      }
    }
  } else {
    constexpr int kChunk = 64 * S;
    const uint8_t* __restrict__ wp = reinterpret_cast<const uint8_t*>(op.w) + wrow_off + kq * 16;
    for (int kc = 0; kc < Kw; kc += kChunk) {
      uint4 q[S];
#pragma unroll
      for (int s = 0; s < S; ++s) q[s] = ld16(wp + kc + s * 64);
      uint4 alo[S], ahi[S];
#pragma unroll
      for (int s = 0; s < S; ++s) fp8x16_to_bf16(q[s], alo[s], ahi[s]);
#pragma unroll
      for (int tb = 0; tb < TOKB; ++tb) {
        if (tb < ntb) {
          const uint16_t* xp = xin + brow[tb] + kq * 16 + kc;
          uint4 b[2 * S];
#pragma unroll
          for (int s = 0; s < S; ++s) {
            b[2 * s] = ld16(xp + s * 64);
            b[2 * s + 1] = ld16(xp + s * 64 + 8);
          }
#pragma unroll
          for (int s = 0; s < S; ++s) {
            acc[tb] = mfma16x16x32(alo[s], b[2 * s], acc[tb]);
            acc[tb] = mfma16x16x32(ahi[s], b[2 * s + 1], acc[tb]);
          }
        }
      }
    }
  }

  // K-split reduction through LDS, summed in wk order by the wk == 0 wave.
  if (WK > 1) {
    if (wk > 0) {
#pragma unroll
      for (int tb = 0; tb < TOKB; ++tb)
        if (tb < ntb) red[(((wk - 1) * WR + wr) * TOKB + tb) * kWave + lane] = acc[tb];
    }
    __syncthreads();
    if (wk > 0) return;
#pragma unroll
    for (int v = 1; v < WK; ++v)
#pragma unroll
      for (int tb = 0; tb < TOKB; ++tb)
        if (tb < ntb) acc[tb] += red[(((v - 1) * WR + wr) * TOKB + tb) * kWave + lane];
  }

  // Epilogue. Lane (q = lane / 16, j = lane % 16) holds rows 4q..4q+3 of token column j.
  const int q = kq;
  const int j = lr;
  const float* sc = op.scale ? op.scale + (long long)(routed ? e : 0) * op.sstride : nullptr;
#pragma unroll
  for (int tb = 0; tb < TOKB; ++tb) {
    if (tb >= ntb) break;
    f32x4_t v = acc[tb];
    int rr = r0 + tb * 16 + j;
    if (MODE == kModeSwiglu) {
      f32x4_t up;
      up[0] = __shfl_down(v[0], 32);
      up[1] = __shfl_down(v[1], 32);
      up[2] = __shfl_down(v[2], 32);
      up[3] = __shfl_down(v[3], 32);
      if (q >= 2 || rr >= r1) continue;
      int n = obase + 4 * q;
      float o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float g = v[i], u = up[i];
        if (sc) {
          g *= sc[n + i];
          u *= sc[op.s_up_off + n + i];
        }
        g = rbf(g);
        u = rbf(u);
        float a = rbf(siluf_(g));
        o[i] = a * u;
      }
      long long orow = routed ? (op.out_map ? args.order[rr] : rr) : rr - args.P;
      uint2 pk = make_uint2(pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3]));
      *reinterpret_cast<uint2*>(op.out + orow * op.ld_out + n) = pk;
    } else {
      if (rr >= r1) continue;
      int n = obase + 4 * q;
      float o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = sc ? v[i] * sc[n + i] : v[i];
      long long orow = routed ? (op.out_map ? args.order[rr] : rr) : rr - args.P;
      uint2 pk = make_uint2(pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3]));
      *reinterpret_cast<uint2*>(op.out + orow * op.ld_out + n) = pk;
    }
  }
}

// ------------------------------------------------------------------------ dispatch

struct StreamCfg {
  int wr, wk, s;
};

template <int MODE, bool HAS_FP8>
static hipError_t launch_cfg(const StreamCfg& c, const GemmArgs& a, int grid, hipStream_t st) {
#define MOE_L(WR, WK, S)                                                                       \
  if (c.wr == WR && c.wk == WK && c.s == S) {                                                  \
    hipLaunchKernelGGL((k_stream_gemm<MODE, WR, WK, S, 4, HAS_FP8>), dim3(grid), dim3(64 * WR * WK), 0, \
                       st, a);                                                                 \
    return hipGetLastError();                                                                  \
  }
  MOE_L(1, 8, 8)
  MOE_L(1, 4, 16)
  MOE_L(1, 4, 8)
  MOE_L(1, 4, 4)
  MOE_L(4, 1, 16)
  MOE_L(4, 1, 8)
  MOE_L(4, 1, 4)
  MOE_L(2, 2, 4)
  MOE_L(1, 1, 1)
#undef MOE_L
  return hipErrorInvalidConfiguration;
}

static bool cfg_fits(const StreamCfg& c, int mode, const GemmOperand& op) {
  if (op.N <= 0) return true;
  int rows = (mode == kModeSwiglu ? 8 : 16) * c.wr;
  int chunk = (op.fp8 ? 64 : 32) * c.s;
  return op.N % rows == 0 && op.K % (c.wk * chunk) == 0;
}

hipError_t launch_stream_gemm(int mode, int role, const GemmArgs& a_in, int max_tiles,
                              hipStream_t st) {
  GemmArgs a = a_in;
  const bool fp8 = (a.op[0].N > 0 && a.op[0].fp8) || (a.op[1].N > 0 && a.op[1].fp8);
  // Preference lists per role; the first configuration both operands fit is used.
  static const StreamCfg kRouter[] = {{1, 8, 8}, {1, 4, 4}, {1, 1, 1}};
  static const StreamCfg kGateUp[] = {{1, 4, 16}, {1, 4, 8}, {1, 4, 4}, {1, 1, 1}};
  static const StreamCfg kDown[] = {{4, 1, 16}, {4, 1, 8}, {4, 1, 4}, {2, 2, 4}, {1, 1, 1}};
  const StreamCfg* list;
  int n;
  if (role == kRoleRouter) {
    list = kRouter;
    n = 3;
  } else if (role == kRoleGateUp) {
    list = kGateUp;
    n = 4;
  } else {
    list = kDown;
    n = 5;
  }
  const StreamCfg* pick = nullptr;
  for (int i = 0; i < n; ++i) {
    const StreamCfg& c = list[i];
    if (fp8 && c.s == 16) continue;
    if (cfg_fits(c, mode, a.op[0]) && cfg_fits(c, mode, a.op[1])) {
      pick = &list[i];
      break;
    }
  }
  if (!pick) return hipErrorInvalidValue;
  int rows = (mode == kModeSwiglu ? 8 : 16) * pick->wr;
  int nmax = a.op[0].N > a.op[1].N ? a.op[0].N : a.op[1].N;
  a.nrb = nmax / rows;
  if (a.nrb <= 0 || max_tiles <= 0) return hipSuccess;
  long long grid = (long long)max_tiles * a.nrb;
  if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
  if (mode == kModeSwiglu)
    return fp8 ? launch_cfg<kModeSwiglu, true>(*pick, a, (int)grid, st)
               : launch_cfg<kModeSwiglu, false>(*pick, a, (int)grid, st);
  return fp8 ? launch_cfg<kModePlain, true>(*pick, a, (int)grid, st)
             : launch_cfg<kModePlain, false>(*pick, a, (int)grid, st);
}

}  // namespace moe
