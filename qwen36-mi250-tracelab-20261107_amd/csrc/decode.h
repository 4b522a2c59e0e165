// Decode-sized MoE block kernels (decode.hip): T <= kDecMaxTokens tokens in three launches.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moe {

constexpr int kDecMaxTokens = 4;

struct DecodeArgs {
  const uint16_t* x;  // [T, H] bf16
  int T, H, E, k, I, IS;
  const uint16_t* w_pack;  // [n_pack, H] router rows, shared gate row at E (K1)
  int n_pack;
  const void* gate_up;     // [E, 2I, H] bf16 or e4m3
  const float* gu_scale;   // [E, 2I] (e4m3)
  const void* down;        // [E, H, I]
  const float* dn_scale;   // [E, H]
  int fp8;
  const uint16_t *sh_gate, *sh_up, *sh_down;  // shared expert (null: routed experts only)
  int sh_in_gate_up;  // shared gate/up rows in the K2 launch instead of the K1 launch
  const uint16_t* residual;                   // [T, H] or null
  int round_w;
  uint16_t* logits;          // [T, n_pack]: written by K1, read by K2 / K3 (null: ids_in)
  const long long* ids_in;   // [T, k] given routing when logits is null
  long long* idx64;          // optional routing output
  int* idx32;                // [T, k] routing for K3 (written by K2)
  uint16_t* wts;             // [T, k] bf16 routing weights (written by K2 when routing)
  uint16_t* act;             // [T * k, I]
  uint16_t* act_sh;          // [T, IS]
  uint16_t* out;             // [T, H]
  // Optional post-attention add + RMSNorm inside K1 (norm_x non-null): K1 computes
  // x = RMSNorm(norm_x + norm_h) itself and its workgroup 0 writes norm_sum (when norm_h)
  // and norm_out, which K2 reads as x and K3 as the residual.
  const uint16_t *norm_x, *norm_h, *norm_w;
  float norm_eps;
  uint16_t *norm_sum, *norm_out;
};

bool decode_fits(const DecodeArgs& a);
hipError_t launch_decode_router(const DecodeArgs& a, hipStream_t s);
hipError_t launch_decode_gate_up(const DecodeArgs& a, hipStream_t s);
hipError_t launch_decode_down(const DecodeArgs& a, hipStream_t s);

}  // namespace moe
