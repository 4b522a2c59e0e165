// Grouped MFMA GEMM for prefill-sized batches on gfx950 (subsystems a8, a9, a6).
//
// Same contract as k_expert_gemm (expert_gemm.hip) and the reference's grouped kernels
// (engine/fast/moe_prefill.py:156-257): for a tile of up to 256 sorted rows of ONE expert,
//   SWIGLU: act[r, n]       = bf16(bf16(silu(bf16 g)) * bf16 u)
//   PLAIN:  out[orow(r), n] = bf16(act_or_x[r] . W[e, n])
// but tiled for ~128 tokens per expert: a workgroup computes 256 weight rows x 256 tokens
// with both operands staged in LDS, so every weight byte read from HBM feeds 256 tokens
// and every token byte feeds 256 weight rows.
//
// Layout. 8 waves: wave (wm, wn) owns weight rows [64 wm, 64 wm + 64) and tokens
// [128 wn, 128 wn + 128) of the tile, i.e. 4 x 8 blocks of v_mfma_f32_16x16x32_bf16
// (128 accumulator registers). SWIGLU puts gate rows in blocks 0-1 and the matching up rows
// in blocks 2-3 of a wave, so the epilogue pairs them in registers. K runs in chunks of 64:
// each chunk of A (256 rows x 128 B) and B (256 rows x 128 B) is loaded global -> VGPR ->
// LDS (row pitch 144 B: the 16-lane 16-byte fragment reads hit distinct banks), double
// buffered; the next chunk's loads are in flight while the current one is multiplied.
#include "moe_common.h"
#include "expert_gemm.h"

namespace moe {

namespace {
constexpr int PBM = 256;              // tokens per tile
constexpr int PBN = 256;              // weight rows per workgroup
constexpr int PKC = 64;               // K elements per chunk
constexpr int kPitch = PKC / 8 + 1;   // LDS row pitch in uint4 (144 B)
constexpr int kStageU4 = (PBN + PBM) * kPitch;  // one stage: A rows then B rows
constexpr int kThreads = 512;
constexpr int kLoads = (PBN + PBM) * (PKC / 8) / kThreads;  // 16-byte loads per thread/chunk
}  // namespace

template <int MODE>
__global__ __launch_bounds__(kThreads, 1) void k_prefill_gemm(GemmArgs args) {
  extern __shared__ uint4 smem[];  // [2][kStageU4]

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
  const int wave = tid >> 6;
  const int wm = wave & 3;   // weight-row group (64 rows)
  const int wn = wave >> 2;  // token group (128 tokens)
  const int lr = lane & 15;
  const int kq = lane >> 4;
  const int nch = op.K / PKC;
  const int ntok = r1 - r0;

  // ---- this thread's 16-byte loads: entry i -> LDS row (A rows 0..255, then B rows).
  const uint16_t* __restrict__ gsrc[kLoads];
  int ldst[kLoads];
  const uint16_t* __restrict__ wbase =
      reinterpret_cast<const uint16_t*>(op.w) + (long long)(routed ? e : 0) * op.estride;
#pragma unroll
  for (int i = 0; i < kLoads; ++i) {
    const int idx = i * kThreads + tid;
    const int row = idx >> 3;  // 8 loads of 16 B per 128-byte row chunk
    const int c = idx & 7;
    ldst[i] = row * kPitch + c;
    if (row < PBN) {
      long long wrow;
      if (MODE == kModeSwiglu) {
        const int g = rb * (PBN / 2) + (row >> 6) * 32 + (row & 31);  // gate row index
        wrow = (long long)g * op.ldw + (((row >> 5) & 1) ? op.up_off : 0);
      } else {
        wrow = (long long)(rb * PBN + row) * op.ldw;
      }
      gsrc[i] = wbase + wrow + c * 8;
    } else {
      const int b = row - PBN;
      int r = min(r0 + b, r1 - 1);
      long long src;
      if (!routed)
        src = r - args.P;
      else if (op.in_map)
        src = args.order[r] / args.topk;
      else
        src = r;
      gsrc[i] = op.in + src * op.ld_in + c * 8;
    }
  }

  uint4 pre[kLoads];
#pragma unroll
  for (int i = 0; i < kLoads; ++i) pre[i] = ld16(gsrc[i]);
#pragma unroll
  for (int i = 0; i < kLoads; ++i) smem[ldst[i]] = pre[i];
  __syncthreads();

  f32x4_t acc[4][8];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 8; ++b) acc[a][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // token blocks of this wave that hold at least one real token
  const int ntb = min(8, max(0, (ntok - wn * 128 + 15) >> 4));

  for (int c = 0; c < nch; ++c) {
    const uint4* st = smem + (c & 1) * kStageU4;
    if (c + 1 < nch) {
#pragma unroll
      for (int i = 0; i < kLoads; ++i) pre[i] = ld16(gsrc[i] + (c + 1) * PKC);
    }
    if (ntb > 0) {
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        uint4 af[4];
#pragma unroll
        for (int a = 0; a < 4; ++a) af[a] = st[(wm * 64 + a * 16 + lr) * kPitch + s * 4 + kq];
#pragma unroll
        for (int b = 0; b < 8; ++b) {
          if (b < ntb) {
            uint4 bf = st[(PBN + wn * 128 + b * 16 + lr) * kPitch + s * 4 + kq];
#pragma unroll
            for (int a = 0; a < 4; ++a) acc[a][b] = mfma16x16x32(af[a], bf, acc[a][b]);
          }
        }
      }
    }
    if (c + 1 < nch) {
      uint4* nx = smem + ((c + 1) & 1) * kStageU4;
#pragma unroll
      for (int i = 0; i < kLoads; ++i) nx[ldst[i]] = pre[i];
    }
    __syncthreads();
  }

  // ---- epilogue: lane (q = kq, j = lr) holds rows 4q..4q+3 of token column j per block.
  const float* sc = op.scale ? op.scale + (long long)(routed ? e : 0) * op.sstride : nullptr;
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    if (b >= ntb) break;
    const int rr = r0 + wn * 128 + b * 16 + lr;
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
  const int out_per_wg = mode == kModeSwiglu ? PBN / 2 : PBN;
  return !op.fp8 && op.N % out_per_wg == 0 && op.K % PKC == 0;
}

hipError_t launch_prefill_gemm(int mode, const GemmArgs& a_in, int max_tiles, hipStream_t st) {
  GemmArgs a = a_in;
  if (!prefill_fits(mode, a.op[0]) || !prefill_fits(mode, a.op[1])) return hipErrorInvalidValue;
  const int out_per_wg = mode == kModeSwiglu ? PBN / 2 : PBN;
  const int nmax = a.op[0].N > a.op[1].N ? a.op[0].N : a.op[1].N;
  a.nrb = nmax / out_per_wg;
  if (a.nrb <= 0 || max_tiles <= 0) return hipSuccess;
  const size_t lds = 2 * (size_t)kStageU4 * sizeof(uint4);
  const long long grid = (long long)max_tiles * a.nrb;
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
