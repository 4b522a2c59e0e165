// Expert-grouped MFMA GEMM for gfx950 with weights streamed from HBM and token rows staged
// through LDS (subsystems a1, a4, a5, a6, a8, a9, a12).
//
// One kernel serves every projection of the MoE block:
//   * router logits        out[t, n]  = bf16(x_t . Wr[n])                 (PLAIN)
//   * expert gate_up       act[r, n]  = bf16(bf16(silu(bf16 g)) * bf16 u)  (SWIGLU)
//                          g = x_tok(r) . Wg[e, n], u = x_tok(r) . Wu[e, n]
//   * expert down          y[pair(r), n] = bf16(act[r] . Wd[e, n])          (PLAIN)
// The rounding points are those of Transformers' batched_mm experts path
// (transformers/integrations/moe.py:112-176), of engine/fast/kernels.py:88-164 and of the
// grouped kernels engine/fast/moe_prefill.py:156-257.
//
// Work decomposition. The sort kernel groups the (token, expert) pairs by expert into
// tiles of up to BM = 16 * TOKB sorted rows of ONE expert (the tile table). A workgroup
// takes one tile and one block of weight rows; every weight element of the block is read
// from HBM once per tile and multiplied against all of the tile's tokens (expert
// de-duplication across the batch).
//
// A workgroup has WR x WK waves. Wave (wr, wk) owns 16 weight rows (SWIGLU: 8 gate rows and
// the matching 8 up rows, paired in registers by the epilogue) and the wk-th of WK slices
// of K; the K partial sums are reduced through LDS in a fixed order (deterministic).
// * A operand (weights): straight from HBM into registers in the v_mfma_f32_16x16x32_bf16
//   A layout (lane = row l%16, 8 consecutive k at 8*(l/16)); 64 contiguous bytes of each of
//   16 rows per load instruction; a ring of NA chunks of KC k-values is kept in flight.
// * B operand (token rows): the WR waves of a K slice stage each chunk of the tile's token
//   rows in LDS with row-contiguous 256-byte loads (four rows per instruction), double
//   buffered, and read it back in the MFMA B layout (row pitch padded by 16-32 bytes).
// fp8-e4m3 weights (per-output-row fp32 scales) are converted to bf16 in registers (exact)
// and the scale multiplies the fp32 accumulator before the bf16 rounding:
// sum_k s_n q_nk x_k = s_n sum_k q_nk x_k.
#include "moe_common.h"
#include "expert_gemm.h"
#include "route_sort_dev.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

namespace moe {

// KC: K elements per chunk (128; 32 for small test shapes, bf16 only); R: chunks in flight.
// One workgroup's tile (expert e, sorted rows [r0, r1), weight-row block rb) with weights of
// one type: HAS_FP8 here means the operand's weights are e4m3.
template <int MODE, int WR, int WK, int TOKB, bool HAS_FP8, int KC, int R>
__device__ __forceinline__ void gemm_tile(const GemmArgs& args, uint4* __restrict__ lds, int e,
                                          int r0, int r1, int rb) {
  constexpr int kRowU4 = KC / 8;        // uint4 per staged token-row chunk (bf16)
  // LDS row pitch in 16-byte units: 2 more than the row, so that it is 2 mod 4. Measured on
  // gfx950 with a one-wave probe of the MFMA B read (lane: row l % 16, unit kq = l / 16):
  // conflict-free for pitches 10, 14, 18, 22, 26, 34, 42 units, 3.8 conflict cycles per
  // ds_read_b128 for every odd pitch and every multiple of 4 (11-26 for multiples of 8), and
  // for any pitch when a k-step's units are not consecutive across kq (see ppart below).
  constexpr int kPitchU4 = kRowU4 + 2;
  constexpr int LPC16 = KC / 32;        // bf16 weight loads per lane per chunk
  constexpr int LPC8 = KC / 64;         // fp8 weight loads per lane per chunk
  constexpr int LPCA = HAS_FP8 ? LPC8 : LPC16;  // ring entries per chunk (16-byte loads)
  static_assert(!HAS_FP8 || LPC8 >= 1, "fp8 needs KC >= 64");
  constexpr int kOutRowsPerWG = (MODE == kModeSwiglu ? 8 : 16) * WR;
  constexpr int BM = 16 * TOKB;
  constexpr int LPR = kRowU4;                  // staging lanes per token row
  constexpr int RPI = 64 / LPR;                // token rows per staging instruction
  constexpr int STG = (TOKB * 16) / (RPI * WR);  // staging instructions per wave per chunk
  static_assert(STG >= 1 && STG * RPI * WR == TOKB * 16, "staging split");
  constexpr int kBufU4 = TOKB * 16 * kPitchU4;  // one chunk of one K slice
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
  const int nch = Kw / KC;
  const int ntb = (r1 - r0 + 15) >> 4;
  constexpr bool use_fp8 = HAS_FP8;

  // ---- A operand: this lane's weight row, first NA chunks requested at once.
  long long wrow_off;
  int obase;  // first output row (PLAIN) / gate row (SWIGLU) of the wave
  if (MODE == kModeSwiglu) {
    obase = rb * kOutRowsPerWG + wr * 8;
    wrow_off = (long long)(obase + (lr & 7)) * op.ldw + (lr >= 8 ? op.up_off : 0);
  } else {
    obase = rb * kOutRowsPerWG + wr * 16;
    wrow_off = (long long)(obase + lr) * op.ldw;
  }
  wrow_off += (long long)(routed ? e : 0) * op.estride + kbeg;
  const uint16_t* __restrict__ wp16 = reinterpret_cast<const uint16_t*>(op.w) + wrow_off + kq * 8;
  const uint8_t* __restrict__ wp8 = reinterpret_cast<const uint8_t*>(op.w) + wrow_off + kq * 16;

  // ---- B staging: this lane moves 16 bytes of STG token rows per chunk into LDS.
  // Staging row q = (i * WR + wr) * RPI + lane / LPR, part = lane % LPR (i < STG).
  const int part = lane % LPR;
  const int qlane = lane / LPR;
  long long srow[STG];
#pragma unroll
  for (int i = 0; i < STG; ++i) {
    int q = (i * WR + wr) * RPI + qlane;
    srow[i] = min(r0 + q, r1 - 1);
  }

  // The weights of the first chunk are requested before the token-row lookups: they depend
  // only on the tile, so their HBM latency overlaps the lookups.
  uint4 aring[R][LPCA];
  if (!use_fp8) {
#pragma unroll
    for (int s = 0; s < LPC16; ++s) aring[0][s] = ld16(wp16 + s * 32);
  } else if (HAS_FP8) {
#pragma unroll
    for (int s = 0; s < LPC8; ++s) aring[0][s] = ld16(wp8 + s * 64);
  }

  if (!routed) {
#pragma unroll
    for (int i = 0; i < STG; ++i) srow[i] -= args.P;
  } else if (op.in_map) {
#pragma unroll
    for (int i = 0; i < STG; ++i) srow[i] = args.order[srow[i]];
#pragma unroll
    for (int i = 0; i < STG; ++i) srow[i] /= args.topk;
  }
  const uint16_t* __restrict__ xin = op.in;
#pragma unroll
  for (int i = 0; i < STG; ++i) srow[i] = srow[i] * op.ld_in + kbeg + part * 8;
  bool sneed[STG];
#pragma unroll
  for (int i = 0; i < STG; ++i) sneed[i] = (i * WR + wr) * RPI + qlane < r1 - r0;
  // Only the tile's real token rows are staged: the LDS rows past them keep stale data,
  // which reaches only MFMA output columns that are never stored.
  uint4* bsl = lds + wk * 2 * kBufU4;  // this K slice's two buffers
  // fp8 tiles: the k-steps read token units 8 s + 2 kq + h (h = 0, 1: the two halves of a
  // lane's 16 weight bytes); each is stored at 8 s + 4 h + kq, so that one k-step's reads
  // are consecutive units across kq, as in the bf16 tiles (read at 8 s + 2 kq + h directly,
  // each read costs 3.8 bank-conflict cycles at any pitch)
  const int ppart = use_fp8 ? ((part & ~7) | ((part & 1) << 2) | ((part >> 1) & 3)) : part;
  auto stage_slot = [&](int i) { return ((i * WR + wr) * RPI + qlane) * kPitchU4 + ppart; };

  // Load stream per chunk m (vmcnt retires in order): A(m) then B(m + 1), each issued R
  // chunks ahead, so waiting for one chunk's data never drains the rest of the ring.
  uint4 bring[R][STG];
  {
    uint4 b0[STG];
#pragma unroll
    for (int i = 0; i < STG; ++i)
      if (sneed[i]) b0[i] = ld16(xin + srow[i]);
#pragma unroll
    for (int m = 0; m < R; ++m) {
      if (m > 0 && m < nch) {
        if (!use_fp8) {
#pragma unroll
          for (int s = 0; s < LPC16; ++s) aring[m][s] = ld16(wp16 + m * KC + s * 32);
        } else if (HAS_FP8) {
#pragma unroll
          for (int s = 0; s < LPC8; ++s) aring[m][s] = ld16(wp8 + m * KC + s * 64);
        }
      }
      if (m + 1 < nch) {
#pragma unroll
        for (int i = 0; i < STG; ++i)
          if (sneed[i]) bring[(m + 1) % R][i] = ld16(xin + srow[i] + (m + 1) * KC);
      }
    }
#pragma unroll
    for (int i = 0; i < STG; ++i)
      if (sneed[i]) bsl[stage_slot(i)] = b0[i];
  }
  __syncthreads();

  f32x4_t acc[TOKB];
#pragma unroll
  for (int tb = 0; tb < TOKB; ++tb) acc[tb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // ---- main loop over chunks; ring slot = chunk % R
  for (int c0 = 0; c0 < nch; c0 += R) {
#pragma unroll
    for (int cc = 0; cc < R; ++cc) {
      const int c = c0 + cc;
      if (c >= nch) break;
      const uint4* bcur = bsl + (c & 1) * kBufU4;
      // one ring entry at a time (bf16: one k-step; fp8: 16 bytes -> two k-steps), so only
      // the fragments of that entry are live
#pragma unroll
      for (int s = 0; s < LPCA; ++s) {
        uint4 a0, a1;
        if (use_fp8)
          fp8x16_to_bf16(aring[cc][s], a0, a1);
        else
          a0 = aring[cc][s];
#pragma unroll
        for (int tb = 0; tb < TOKB; ++tb) {
          if (tb < ntb) {
            const uint4* brow = bcur + (tb * 16 + lr) * kPitchU4;
            if (use_fp8) {
              // fp8 A lane kq holds k = s*64 + kq*16 + h*8 (+0..7): token unit 8 s + 2 kq + h,
              // stored at 8 s + 4 h + kq
              acc[tb] = mfma16x16x32(a0, brow[s * 8 + kq], acc[tb]);
              acc[tb] = mfma16x16x32(a1, brow[s * 8 + 4 + kq], acc[tb]);
            } else {
              acc[tb] = mfma16x16x32(a0, brow[s * 4 + kq], acc[tb]);
            }
          }
        }
      }
      // next chunk's token rows into the other LDS buffer
      if (c + 1 < nch) {
        uint4* bnext = bsl + ((c + 1) & 1) * kBufU4;
#pragma unroll
        for (int i = 0; i < STG; ++i)
          if (sneed[i]) bnext[stage_slot(i)] = bring[(cc + 1) % R][i];
      }
      // refill: A(c + R) into this slot, B(c + 1 + R) into the slot just drained
      if (c + R < nch) {
        if (!use_fp8) {
#pragma unroll
          for (int s = 0; s < LPC16; ++s) aring[cc][s] = ld16(wp16 + (c + R) * KC + s * 32);
        } else if (HAS_FP8) {
#pragma unroll
          for (int s = 0; s < LPC8; ++s) aring[cc][s] = ld16(wp8 + (c + R) * KC + s * 64);
        }
      }
      if (c + 1 + R < nch) {
#pragma unroll
        for (int i = 0; i < STG; ++i)
          if (sneed[i]) bring[(cc + 1) % R][i] = ld16(xin + srow[i] + (c + 1 + R) * KC);
      }
      __syncthreads();
    }
  }

  // ---- K-split reduction through LDS (buffers reused), summed in wk order by wk == 0.
  if (WK > 1) {
    f32x4_t* red = reinterpret_cast<f32x4_t*>(lds);
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

  // ---- epilogue. Lane (q = lane / 16, j = lane % 16) holds rows 4q..4q+3 of token column j.
  const int q = kq;
  const int j = lr;
  const float* sc = op.scale ? op.scale + (long long)(routed ? e : 0) * op.sstride : nullptr;
#pragma unroll
  for (int tb = 0; tb < TOKB; ++tb) {
    if (tb >= ntb || wk > 0) break;
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

// Waves per SIMD the compiler must allow: three for tiles of up to 32 tokens, unless the
// configuration's rings (A chunks in flight plus staged token rows) need 96 or more VGPRs,
// where the 168-register cap of three waves made the compiler spill; two then.
constexpr int gemm_waves_per_eu(int WR, int TOKB, bool fp8, int KC, int R) {
  const int lpca = fp8 ? KC / 64 : KC / 32;
  const int stg = (TOKB * 16) / ((64 / (KC / 8)) * WR);
  const int ring = 4 * R * (lpca + stg);
  return TOKB <= 2 && KC >= 64 ? (ring >= 96 ? 2 : 3) : 1;
}

// The kernel: looks up its tile and runs it with the tile's weight type. An fp8 launch may
// also hold bf16 tiles (the shared expert beside fp8 routed experts): those run with half
// the chunk length, which gives them the fp8 tiles' ring of A registers.
template <int MODE, int WR, int WK, int TOKB, bool HAS_FP8, int KC, int R = 4>
__global__ __launch_bounds__(64 * WR * WK)
__attribute__((amdgpu_waves_per_eu(gemm_waves_per_eu(WR, TOKB, HAS_FP8, KC, R))))
void k_expert_gemm(GemmArgs args) {
  constexpr int kRowU4 = KC / 8;
  constexpr int kPitchU4 = kRowU4 + 2;
  constexpr int kBufU4 = TOKB * 16 * kPitchU4;
  constexpr int BM = 16 * TOKB;
  // LDS: [WK][2 buffers][TOKB*16 rows][pitch] uint4 at this KC (the larger of the two
  // bodies'); reused for the K-split reduction.
  __shared__ uint4 lds[WK * 2 * kBufU4];


  const int nrb = args.nrb;
  int tile = blockIdx.x / nrb;
  const int rb = blockIdx.x - tile * nrb;

  int e, r0, r1;
  if (args.table) {
    const int ntiles = args.table[3 * args.MT];
    if (tile >= ntiles) return;
    if (args.shared_first > 0) {
      // the shared expert's tiles (the table's last ones: every token of the batch, and in
      // an fp8 launch bf16 rows of twice the bytes) are dispatched first, so that the
      // longest workgroups do not start in the launch's last round
      const int ns = min(args.shared_first, ntiles);
      tile = tile < ns ? ntiles - ns + tile : tile - ns;
    }
    e = args.table[tile];
    r0 = args.table[args.MT + tile];
    r1 = args.table[2 * args.MT + tile];
  } else {
    e = args.E;
    r0 = args.P + tile * BM;
    if (r0 >= args.P + args.T) return;
    r1 = min(r0 + BM, args.P + args.T);
  }
  if constexpr (HAS_FP8) {
    if ((e < args.E ? args.op[0] : args.op[1]).fp8)
      gemm_tile<MODE, WR, WK, TOKB, true, KC, R>(args, lds, e, r0, r1, rb);
    else
      gemm_tile<MODE, WR, WK, TOKB, false, KC / 2, R>(args, lds, e, r0, r1, rb);
  } else {
    gemm_tile<MODE, WR, WK, TOKB, false, KC, R>(args, lds, e, r0, r1, rb);
  }
}

// ------------------------------------------------------------------------ dispatch

namespace {

struct Cfg {
  int wr, wk, tokb, kc, r = 4;  // r: chunks in flight
};

template <int MODE, bool HAS_FP8>
hipError_t launch_cfg(const Cfg& c, const GemmArgs& a, int grid, hipStream_t st) {
#define MOE_LAUNCH(WR, WK, TOKB, KCV, RV)                                                       \
  hipLaunchKernelGGL((k_expert_gemm<MODE, WR, WK, TOKB, HAS_FP8, KCV, RV>), dim3(grid),         \
                     dim3(64 * WR * WK), 0, st, a);                                             \
  return hipGetLastError();
#define MOE_L(WR, WK, TOKB, KCV, RV)                                                            \
  if (c.wr == WR && c.wk == WK && c.tokb == TOKB && c.kc == KCV && c.r == RV) {                \
    MOE_LAUNCH(WR, WK, TOKB, KCV, RV)                                                           \
  }
  // the configurations the preference lists of launch_expert_gemm can reach
  if constexpr (HAS_FP8) {
    MOE_L(4, 1, 2, 256, 2)
    MOE_L(4, 1, 2, 128, 4)
    MOE_L(2, 1, 2, 128, 4)
    MOE_L(1, 4, 1, 64, 8)
    MOE_L(1, 2, 1, 128, 4)
    MOE_L(1, 1, 1, 128, 4)
    MOE_L(4, 1, 4, 64, 8)
    MOE_L(4, 1, 8, 64, 4)
  } else {
    MOE_L(1, 8, 1, 64, 4)
    MOE_L(1, 4, 1, 64, 4)
    MOE_L(2, 2, 2, 64, 4)
    MOE_L(2, 1, 2, 64, 4)
    MOE_L(4, 1, 4, 64, 4)
    MOE_L(4, 1, 8, 64, 4)
    MOE_L(1, 2, 1, 128, 4)
    MOE_L(1, 1, 1, 128, 4)
    MOE_L(2, 1, 2, 128, 4)
    MOE_L(1, 1, 1, 32, 4)
    MOE_L(1, 1, 2, 32, 4)
    MOE_L(1, 1, 4, 32, 4)
  }
#undef MOE_L
#undef MOE_LAUNCH
  return hipErrorInvalidConfiguration;
}

bool fits(const Cfg& c, int mode, const GemmOperand& op) {
  if (op.N <= 0) return true;
  int rows = (mode == kModeSwiglu ? 8 : 16) * c.wr;
  if (op.fp8 && c.kc < 64) return false;
  return op.N % rows == 0 && op.K % (c.wk * c.kc) == 0;
}

}  // namespace

bool mixed_enabled() {
  const char* env = knob(kKnobMixed);
  return !(env && env[0] == '0');
}

hipError_t launch_expert_gemm(int mode, int role, int bm, const GemmArgs& a_in, int max_tiles,
                              hipStream_t st) {
  GemmArgs a = a_in;
  const bool fp8 = (a.op[0].N > 0 && a.op[0].fp8) || (a.op[1].N > 0 && a.op[1].fp8);
  // an fp8 launch may hold bf16 tiles (they run at half the chunk length); a launch of
  // bf16 configurations cannot hold fp8 tiles
  if (a.op[0].N > 0 && a.op[1].N > 0 && a.op[0].fp8 != a.op[1].fp8 && !mixed_enabled())
    return hipErrorInvalidValue;
  const int tokb = bm / 16;
  if (bm % 16 || (tokb != 1 && tokb != 2 && tokb != 4 && tokb != 8)) return hipErrorInvalidValue;
  // Preferences: with one 16-token block per tile, split K over 4 waves (more waves for the
  // few-token decode case); with 4 blocks, 4 row groups share the staged token rows.
  Cfg prefs[8];
  int n = 0;
  // fp8 weights move half the bytes per K element: 128-element chunks keep as many bytes
  // in flight as the bf16 64-element ones.
  const int rr = fp8 ? 8 : 4;  // fp8: 64-element chunks are half the bytes, twice as many
  if (role == kRoleRouter && tokb == 1 && !fp8) prefs[n++] = {1, 8, 1, 64, rr};
  if (tokb == 1) {
    prefs[n++] = {1, 4, 1, 64, rr};
    prefs[n++] = {1, 2, 1, 128};
    prefs[n++] = {1, 1, 1, 128};
  } else if (tokb == 2) {
    if (fp8) {
      // fp8 32-token tiles: four row groups per workgroup; gate_up with 128-element chunks
      // four deep, down (K = 512) with 256-element chunks two deep (the fastest measured at
      // the 40-layer T=32 shape: 157 against 161 µs per layer with 256 x 2 for gate_up)
      if (role == kRoleDown) {
        prefs[n++] = {4, 1, 2, 256, 2};
        prefs[n++] = {4, 1, 2, 128, 4};
      } else {
        prefs[n++] = {4, 1, 2, 128, 4};
        prefs[n++] = {4, 1, 2, 256, 2};
      }
    } else {
      prefs[n++] = role == kRoleDown ? Cfg{2, 1, 2, 64, rr} : Cfg{2, 2, 2, 64, rr};
    }
    prefs[n++] = {2, 1, 2, 128};
  } else if (tokb == 4) {
    prefs[n++] = {4, 1, 4, 64, rr};
  } else {
    prefs[n++] = {4, 1, 8, 64};
  }
  prefs[n++] = {1, 1, tokb, 32};  // small test shapes (K a multiple of 32)
  for (int i = 0; i < n; ++i) {
    const Cfg& c = prefs[i];
    if (!fits(c, mode, a.op[0]) || !fits(c, mode, a.op[1])) continue;
    if (c.wk * 2 * c.tokb * 16 * (c.kc / 8 + 2) * 16 > 65536) continue;
    int rows = (mode == kModeSwiglu ? 8 : 16) * c.wr;
    int nmax = a.op[0].N > a.op[1].N ? a.op[0].N : a.op[1].N;
    a.nrb = nmax / rows;
    if (a.nrb <= 0 || max_tiles <= 0) return hipSuccess;
    a.shared_first = 0;
    if (a.table && a.op[0].N > 0 && a.op[1].N > 0) {
      const char* env = knob(kKnobGemmSharedFirst);
      if (!(env && env[0] == '0')) a.shared_first = (a.T + c.tokb * 16 - 1) / (c.tokb * 16);
    }
    long long grid = (long long)max_tiles * a.nrb;
    if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
    hipError_t err;
    if (mode == kModeSwiglu)
      err = fp8 ? launch_cfg<kModeSwiglu, true>(c, a, (int)grid, st)
                : launch_cfg<kModeSwiglu, false>(c, a, (int)grid, st);
    else
      err = fp8 ? launch_cfg<kModePlain, true>(c, a, (int)grid, st)
                : launch_cfg<kModePlain, false>(c, a, (int)grid, st);
    if (err == hipErrorInvalidConfiguration) continue;  // not instantiated: next choice
    return err;
  }
  return hipErrorInvalidValue;
}

}  // namespace moe
