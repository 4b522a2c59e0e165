// Arguments of the expert-grouped MFMA GEMM (expert_gemm.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moe {

constexpr int kModePlain = 0;   // out = bf16(acc * scale)
constexpr int kModeSwiglu = 1;  // out = bf16(bf16(silu(bf16 g)) * bf16 u), gate/up row pairs

constexpr int kRoleRouter = 0;
constexpr int kRoleGateUp = 1;
constexpr int kRoleDown = 2;

// One weight family: the routed experts (op[0]) or the virtual expert id E (op[1],
// the shared expert or the router), whose rows map 1:1 to tokens (row r -> token r - P).
struct GemmOperand {
  const void* w;        // expert 0, output row 0 (SWIGLU: gate row 0); bf16 or fp8 elements
  long long estride;    // elements between experts
  long long up_off;     // SWIGLU: elements from gate row n to up row n
  long long ldw;        // elements per weight row
  const float* scale;   // per-output-row fp32 scales (fp8) or null
  long long sstride;    // scales per expert
  long long s_up_off;   // SWIGLU: scale index of up row 0
  int K, N;             // reduction length; output rows (SWIGLU: gate rows)
  const uint16_t* in;   // B operand rows (bf16)
  long long ld_in;
  uint16_t* out;        // bf16 output rows
  long long ld_out;
  int in_map;           // routed: 1 -> B row = token of pair order[r]; 0 -> B row = r
  int out_map;          // routed: 1 -> out row = pair order[r]; 0 -> out row = r
  int fp8;              // weights are OCP e4m3fn bytes (else bf16)
};

struct GemmArgs {
  GemmOperand op[2];
  const int* table;  // tile table, or null: virtual-expert tiles over rows P .. P + T
  int MT;            // table capacity (max tiles)
  const int* order;  // sorted row -> pair
  int topk, P, E, T;
  int nrb;           // weight-row blocks per tile (set by the launcher)
  int MTgrid;        // tiles the grid covers (set by the launcher)
  int shared_first;  // the table's last shared_first tiles run first (set by the launcher)
};

// Launches k_expert_gemm over max_tiles tiles of at most bm (16, 32, 64 or 128) sorted rows.
// Both operands of one launch must have the same weight type.
// hipErrorInvalidValue: no kernel configuration fits the operands' shapes.
// Whether a launch may mix fp8 routed tiles with bf16 shared-expert tiles (MOE_MIXED=0: no;
// then the caller splits them into two launches).
bool mixed_enabled();
hipError_t launch_expert_gemm(int mode, int role, int bm, const GemmArgs& a, int max_tiles,
                              hipStream_t st);

// Prefill tiles (prefill_gemm.hip): 256 sorted rows x 256 weight rows per workgroup, bf16.
int prefill_tile_rows();
bool prefill_fits(int mode, const GemmOperand& op);
hipError_t launch_prefill_gemm(int mode, const GemmArgs& a, int max_tiles, hipStream_t st);

}  // namespace moe
