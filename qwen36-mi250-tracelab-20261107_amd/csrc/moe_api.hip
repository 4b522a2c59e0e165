// extern "C" entry points of libmoe_mi355x.so (declared in include/moe_mi355x.h).
// Validation, workspace carving and the launch sequence of the MoE block; the kernels
// live in route_sort.hip, expert_gemm.hip, prefill_gemm.hip, decode.hip, add_rms.hip and
// combine.hip.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <mutex>
#include <string>

#include "../../include/moe_mi355x.h"
#include "add_rms.h"
#include "expert_gemm.h"
#include "decode.h"

namespace moe {
hipError_t launch_route(const uint16_t* logits, long long ld, int T, int E, int k, long long* idx64,
                        int* idx32, uint16_t* w_out, int* counts, hipStream_t s);
hipError_t launch_route_sort(const uint16_t* logits, long long ld, const int* ids32_in,
                             const long long* ids64_in, int T, int E, int k, int bm, int has_shared,
                             long long* idx64, int* idx32, uint16_t* w_out, int* counts,
                             int* offsets, int* order, int* table, int MT, int* scratch,
                             hipStream_t s);
size_t sort_scratch_bytes(int P, int E);
bool sort_uses_small(int P, int E);
bool router_gemm_fits(int H, int n_pack);
bool router_part_takes(int T, int H, int n_pack);
hipError_t launch_router_part(const void* x, int T, int H, const void* w_pack, int n_pack,
                              float* part, hipStream_t st);
hipError_t launch_route_part(const float* part, int T, int n_pack, int E, int k,
                             uint16_t* logits, long long* idx64, int* idx32, uint16_t* w_out,
                             hipStream_t s);
hipError_t launch_router_gemm(const void* x, int T, int H, const void* w_pack, int n_pack,
                              void* logits, hipStream_t st);
hipError_t launch_combine(const uint16_t* y, const uint16_t* w, int k, const uint16_t* ysh,
                          const uint16_t* seg, long long ld_seg, const uint16_t* res, uint16_t* out,
                          int T, int H, int round_w, hipStream_t s);
}  // namespace moe

using namespace moe;

namespace {

// Sorted rows per tile of the grouped GEMMs: one 16-row MFMA block for decode-sized batches
// (K split over 4 waves), two blocks up to 512 tokens, and 256-row tiles of the prefill
// kernel above (bf16 weights with shapes it tiles; else 64-row tiles of the expert GEMM).
int tile_rows_for(int T, bool fp8 = false, int H = 2048, int I = 512, int IS = 512) {
  // 32-row tiles from 2 tokens: per layer (12 layers cycled) 8 / 16 tokens take 81 / 113 µs
  // with fp8 experts against 128 / 213 with 16-row tiles, and 102 / 150 against 107 / 166
  // with bf16; at 2 / 3 / 4 tokens (16 layers) fp8 50 / 53 / 56 against 55 / 68 / 79 and
  // bf16 49 / 59 / 69 against 51 / 60 / 69; one token 44 against 40 (bf16)
  if (T <= 1) return 16;
  if (T <= 512) return 32;
  (void)fp8;  // e4m3 experts take the same tiles (prefill_gemm.hip's fp8 kernel)
  const bool prefill_ok = H % 256 == 0 && I % 128 == 0 && IS % 128 == 0;
  return prefill_ok ? prefill_tile_rows() : 64;
}

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_check(hipError_t e, const char* what) {
  if (e == hipSuccess) return MOE_OK;
  return fail(MOE_EHIP, "%s: %s", what, hipGetErrorString(e));
}

#define CHECK_ARG(cond, ...) \
  do {                       \
    if (!(cond)) return fail(MOE_EINVAL, __VA_ARGS__); \
  } while (0)

#define HIP_TRY(expr, what)                     \
  do {                                          \
    int rc_ = hip_check((expr), what);          \
    if (rc_ != MOE_OK) return rc_;              \
  } while (0)

// The three-launch decode path (decode.hip) for T <= 4 unless MOE_DECODE=0.
bool decode_enabled() {
  const char* env = knob(kKnobDecode);
  return !(env && env[0] == '0');
}

// Whether the decode kernels take T tokens (given that the shape fits them): measured per
// layer (16 layers cycled) against the tiled path with 32-row tiles, bf16 decode
// 17.6 / 31.2 / 52.8 / 67.6 µs at 1 / 2 / 3 / 4 tokens against 43.9 / 49.3 / 58.6 / 68.7;
// fp8 at 4 tokens, since the several-row-block gate_up kernel, 47.7-47.9 against 56.9-57.1
// (8 layers cycled): both weight types up to kDecMaxTokens.
bool decode_takes(int T, bool fp8) {
  (void)fp8;
  return decode_enabled() && T <= kDecMaxTokens;
}

// A grouped prefill launch with routed and shared tiles: one launch, the shared expert's
// tiles dispatched first (grouped gate_up at C4 303-310 against 317 µs with the shared
// tiles as a second launch on the auxiliary stream, 632 with them dispatched last);
// MOE_PREFILL_SIDE=1 restores the second launch. (The block forward runs the whole shared
// expert on the auxiliary stream from its start instead; see block_side_enabled.)
bool prefill_side_enabled() {
  const char* env = knob(kKnobPrefillSide);
  return env && env[0] == '1';
}

// Block forward: the shared expert on the auxiliary stream where it runs as separate
// launches anyway: fp8 routed experts whose bf16 shared tiles do not share the routed
// launches (MOE_MIXED=0), or prefill tiles.
bool block_side_enabled(bool fp8, int bm) {
  return (fp8 && !mixed_enabled()) || bm == prefill_tile_rows();
}

size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

// Sequential carve of a caller-provided workspace.
struct Carver {
  char* base;
  size_t off = 0;
  template <class Tp>
  Tp* take(size_t count) {
    Tp* p = base ? reinterpret_cast<Tp*>(base + off) : nullptr;
    off += align256(count * sizeof(Tp));
    return p;
  }
};

int max_tiles_of(int T, int k, int E, int bm, int has_shared) {
  long long P = (long long)T * k;
  long long mt = (P + bm - 1) / bm + (P < E ? P : E);
  if (has_shared) mt += (T + bm - 1) / bm;
  return (int)mt;
}

int check_experts_shape(int T, int H, int E, int k, int I) {
  CHECK_ARG(T >= 0, "T must be >= 0 (got %d)", T);
  CHECK_ARG(E >= 1 && E <= 1024, "experts must be in [1, 1024] (got %d)", E);
  CHECK_ARG(k >= 1 && k <= 64 && k <= E, "top_k must be in [1, min(64, E)] (got %d)", k);
  CHECK_ARG(H >= 32 && H % 32 == 0, "hidden must be a positive multiple of 32 (got %d)", H);
  CHECK_ARG(I >= 32 && I % 32 == 0, "intermediate must be a positive multiple of 32 (got %d)", I);
  CHECK_ARG((long long)T * k < (1LL << 30), "too many pairs");
  return MOE_OK;
}

GemmOperand gate_up_operand(const void* gate_up, const float* scale, int H, int I, const void* in,
                            void* act) {
  GemmOperand o{};
  o.w = gate_up;
  o.estride = 2LL * I * H;
  o.up_off = (long long)I * H;
  o.ldw = H;
  o.scale = scale;
  o.sstride = 2LL * I;
  o.s_up_off = I;
  o.K = H;
  o.N = I;
  o.in = static_cast<const uint16_t*>(in);
  o.ld_in = H;
  o.out = static_cast<uint16_t*>(act);
  o.ld_out = I;
  o.in_map = 1;
  o.out_map = 0;
  return o;
}

GemmOperand down_operand(const void* down, const float* scale, int H, int I, const void* act,
                         void* y) {
  GemmOperand o{};
  o.w = down;
  o.estride = (long long)H * I;
  o.ldw = I;
  o.scale = scale;
  o.sstride = H;
  o.K = I;
  o.N = H;
  o.in = static_cast<const uint16_t*>(act);
  o.ld_in = I;
  o.out = static_cast<uint16_t*>(y);
  o.ld_out = H;
  o.in_map = 0;
  o.out_map = 1;
  return o;
}

// A second stream per device for work that can run beside the caller's stream (forked and
// joined with events, so it is ordered with the caller's work and is captured into the
// caller's HIP graph as a parallel branch). Created on first use outside graph capture;
// while none exists the work runs on the caller's stream. Default priority.
// One stream per device, not one per caller stream: HIP maps streams onto its few hardware
// queues round-robin, and with more streams the side branch can land on the caller's queue
// and lose the overlap (measured at C4: 640 against 600 µs per layer). Calls from several
// threads or caller streams are kept apart by the device's lock, held from fork to join
// (see Fork).
struct AuxStream {
  hipStream_t s = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
  std::recursive_mutex mu;
};
AuxStream* aux_stream(hipStream_t caller) {
  static std::mutex mu;
  static AuxStream per_device[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  AuxStream& a = per_device[dev];
  if (a.s) return &a;
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(caller, &st) != hipSuccess || st != hipStreamCaptureStatusNone)
    return nullptr;
  if (hipStreamCreateWithFlags(&a.s, hipStreamNonBlocking) != hipSuccess) {
    a.s = nullptr;
    return nullptr;
  }
  if (hipEventCreateWithFlags(&a.fork, hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&a.join, hipEventDisableTiming) != hipSuccess) {
    if (a.fork) hipEventDestroy(a.fork);
    hipStreamDestroy(a.s);
    a.s = nullptr;
    return nullptr;
  }
  return &a;
}

// One fork of the caller's stream onto the device's auxiliary stream. It holds the
// auxiliary stream's lock for its lifetime, so the record / wait / launch / record / wait
// sequence of one call never interleaves with another call's (another thread, another
// caller stream) and a fork event is never re-recorded before its wait is queued. The join
// runs on every path out of the scope that forked, errors included, so the caller's stream
// (and a graph being captured on it) never returns with a branch left open.
class Fork {
 public:
  Fork(AuxStream* aux, hipStream_t s) : aux_(aux), s_(s) {
    if (aux_) lock_ = std::unique_lock<std::recursive_mutex>(aux_->mu);
  }
  Fork(const Fork&) = delete;
  Fork& operator=(const Fork&) = delete;
  ~Fork() { (void)join(); }
  // Work queued on aux() after begin() waits for the caller's stream up to here.
  hipError_t begin() {
    if (!aux_) return hipSuccess;
    hipError_t e = hipEventRecord(aux_->fork, s_);
    if (e == hipSuccess) e = hipStreamWaitEvent(aux_->s, aux_->fork, 0);
    open_ = e == hipSuccess;
    return e;
  }
  // The caller's stream waits for the work queued on aux().
  hipError_t join() {
    if (!open_) return hipSuccess;
    open_ = false;
    hipError_t e = hipEventRecord(aux_->join, aux_->s);
    if (e == hipSuccess) e = hipStreamWaitEvent(s_, aux_->join, 0);
    return e;
  }
  hipStream_t aux() const { return aux_ ? aux_->s : s_; }

 private:
  AuxStream* aux_;
  hipStream_t s_;
  std::unique_lock<std::recursive_mutex> lock_;
  bool open_ = false;
};

// Prefill tiles: the routed tiles fill whole rounds of one workgroup per CU (~256 experts x
// 4 or 8 row blocks), and the shared expert's tiles would add a last, mostly idle round; run
// them as a second launch on the auxiliary stream instead, where they fill the gaps of the
// routed launch.
hipError_t launch_prefill_split(int mode, const GemmArgs& a, int MT, hipStream_t s) {
  AuxStream* aux = a.op[0].N > 0 && a.op[1].N > 0 && a.table ? aux_stream(s) : nullptr;
  if (!aux || !prefill_side_enabled()) return launch_prefill_gemm(mode, a, MT, s);
  GemmArgs v = a;  // no table: the prefill kernel reads tile i as shared rows [bm i, bm i + bm)
  v.op[0].N = 0;
  v.table = nullptr;
  Fork fork(aux, s);
  hipError_t e = fork.begin();
  if (e != hipSuccess) return e;
  e = launch_prefill_gemm(mode, v, (a.T + prefill_tile_rows() - 1) / prefill_tile_rows(),
                          fork.aux());
  if (e != hipSuccess) return e;
  GemmArgs r = a;
  r.op[1].N = 0;
  e = launch_prefill_gemm(mode, r, MT, s);
  if (e != hipSuccess) return e;
  return fork.join();
}

// One launch for the routed experts and the shared expert, or two when their weight types
// differ (fp8 experts, bf16 shared expert) and MOE_MIXED=0: then the shared expert's tiles
// come from the token count alone (rows P .. P + T), on the auxiliary stream so that the two
// launches overlap. By default (mixed_enabled) an fp8 launch takes the bf16 tiles itself.
hipError_t launch_split(int mode, int role, int bm, const GemmArgs& a, int MT, hipStream_t s) {
  if (a.op[0].N <= 0 || a.op[1].N <= 0 || a.op[0].fp8 == a.op[1].fp8 || mixed_enabled())
    return launch_expert_gemm(mode, role, bm, a, MT, s);
  GemmArgs v = a;
  v.op[0] = v.op[1];
  v.op[0].N = 0;
  v.table = nullptr;
  Fork fork(aux_stream(s), s);
  hipError_t err = fork.begin();
  if (err != hipSuccess) return err;
  err = launch_expert_gemm(mode, role, bm, v, (a.T + bm - 1) / bm, fork.aux());
  if (err != hipSuccess) return err;
  GemmArgs r = a;
  r.op[1].N = 0;
  err = launch_expert_gemm(mode, role, bm, r, MT, s);
  if (err != hipSuccess) return err;
  return fork.join();
}

// Which projections a grouped launch runs: both weight families (split as above when
// needed), the routed experts only, or the shared expert only (its tiles from the token
// count alone).
enum Part { kBoth = 0, kRoutedOnly = 1, kSharedOnly = 2 };

hipError_t launch_part(int mode, int role, int bm, const GemmArgs& a, int MT, int part,
                       hipStream_t s) {
  const bool prefill = bm == prefill_tile_rows();
  if (part == kRoutedOnly) {
    GemmArgs r = a;
    r.op[1].N = 0;
    return prefill ? launch_prefill_gemm(mode, r, MT, s) : launch_expert_gemm(mode, role, bm, r, MT, s);
  }
  if (part == kSharedOnly) {
    GemmArgs v = a;
    v.table = nullptr;
    const int tiles = (a.T + bm - 1) / bm;
    if (prefill) {
      v.op[0].N = 0;  // the prefill kernel reads tile i as shared rows [bm i, bm i + bm)
      return launch_prefill_gemm(mode, v, tiles, s);
    }
    v.op[0] = v.op[1];  // the configuration follows op[0]'s weight type
    v.op[0].N = 0;
    return launch_expert_gemm(mode, role, bm, v, tiles, s);
  }
  return prefill ? launch_prefill_split(mode, a, MT, s) : launch_split(mode, role, bm, a, MT, s);
}

int run_gate_up(const void* x, int T, int H, int E, int k, int I, const void* gate_up,
                const float* gu_scale, int wdtype, const void* sh_gate, const void* sh_up, int IS,
                const int* order, const int* table, int MT, int bm, void* act, void* act_sh,
                hipStream_t s, int part = kBoth) {
  GemmArgs a{};
  a.op[0] = gate_up_operand(gate_up, gu_scale, H, I, x, act);
  a.op[0].fp8 = wdtype == MOE_WEIGHTS_FP8_E4M3;
  if (sh_gate) {
    GemmOperand& v = a.op[1];
    v.w = sh_gate;
    v.up_off = (long long)((intptr_t)sh_up - (intptr_t)sh_gate) / 2;
    v.ldw = H;
    v.K = H;
    v.N = IS;
    v.in = static_cast<const uint16_t*>(x);
    v.ld_in = H;
    v.out = static_cast<uint16_t*>(act_sh);
    v.ld_out = IS;
  } else {
    a.op[1] = a.op[0];
    a.op[1].N = 0;
  }
  a.table = table;
  a.MT = MT;
  a.order = order;
  a.topk = k;
  a.P = T * k;
  a.E = E;
  a.T = T;
  hipError_t err = launch_part(kModeSwiglu, kRoleGateUp, bm, a, MT, sh_gate ? part : kBoth, s);
  if (err == hipErrorInvalidValue)
    return fail(MOE_EINVAL, "gate_up: no kernel configuration for H=%d I=%d IS=%d", H, I, IS);
  return hip_check(err, "gate_up launch");
}

int run_down(const void* act, int T, int H, int E, int k, int I, const void* down,
             const float* dn_scale, int wdtype, const void* sh_down, int IS, const void* act_sh,
             const int* order, const int* table, int MT, int bm, void* y, void* y_sh,
             hipStream_t s, int part = kBoth) {
  GemmArgs a{};
  a.op[0] = down_operand(down, dn_scale, H, I, act, y);
  a.op[0].fp8 = wdtype == MOE_WEIGHTS_FP8_E4M3;
  if (sh_down) {
    GemmOperand& v = a.op[1];
    v.w = sh_down;
    v.ldw = IS;
    v.K = IS;
    v.N = H;
    v.in = static_cast<const uint16_t*>(act_sh);
    v.ld_in = IS;
    v.out = static_cast<uint16_t*>(y_sh);
    v.ld_out = H;
  } else {
    a.op[1] = a.op[0];
    a.op[1].N = 0;
  }
  a.table = table;
  a.MT = MT;
  a.order = order;
  a.topk = k;
  a.P = T * k;
  a.E = E;
  a.T = T;
  hipError_t err = launch_part(kModePlain, kRoleDown, bm, a, MT, sh_down ? part : kBoth, s);
  if (err == hipErrorInvalidValue)
    return fail(MOE_EINVAL, "down: no kernel configuration for H=%d I=%d IS=%d", H, I, IS);
  return hip_check(err, "down launch");
}

}  // namespace

namespace moe {
namespace {
const char* const kKnobNames[kKnobCount] = {"MOE_DECODE",       "MOE_DECODE_DOWN",
                                            "MOE_DECODE_GU_BLOCKS", "MOE_MIXED",
                                            "MOE_PREFILL_SIDE", "MOE_PREFILL_SHARED_FIRST",
                                            "MOE_GEMM_SHARED_FIRST"};
std::mutex g_knob_mu;
std::atomic<bool> g_knobs_read{false};
char g_knob_val[kKnobCount][32];
bool g_knob_set[kKnobCount];

void read_knobs() {
  std::lock_guard<std::mutex> lock(g_knob_mu);
  for (int i = 0; i < kKnobCount; ++i) {
    const char* v = getenv(kKnobNames[i]);
    g_knob_set[i] = v != nullptr;
    snprintf(g_knob_val[i], sizeof g_knob_val[i], "%s", v ? v : "");
  }
  g_knobs_read.store(true, std::memory_order_release);
}
}  // namespace

const char* knob(Knob k) {
  if (!g_knobs_read.load(std::memory_order_acquire)) read_knobs();
  return g_knob_set[k] ? g_knob_val[k] : nullptr;
}
}  // namespace moe

extern "C" {

int moe_abi_version(void) { return MOE_ABI_VERSION; }


void moe_reload_tuning(void) { read_knobs(); }

const char* moe_last_error(void) { return g_err.c_str(); }

int moe_tile_rows(int T) { return tile_rows_for(T); }

int moe_max_tiles(int T, int k, int E, int bm, int has_shared) {
  if (T < 0 || k < 1 || E < 1 || bm < 1) return 0;
  return max_tiles_of(T, k, E, bm, has_shared);
}

}  // extern "C"

namespace {
// Router GEMM: k_router_gemm (router_gemm.hip), whose per-logit summation order is the same
// at every batch size; shapes it does not take (hidden not a multiple of 128) use the expert
// GEMM's 16-token identity tiles with K split over 8 waves, also one order for every T.
hipError_t launch_router(const void* x, int T, int H, const void* w_pack, int n_pack,
                         void* logits, hipStream_t st) {
  if (router_gemm_fits(H, n_pack)) return launch_router_gemm(x, T, H, w_pack, n_pack, logits, st);
  GemmArgs a{};
  GemmOperand& v = a.op[1];
  v.w = w_pack;
  v.ldw = H;
  v.K = H;
  v.N = n_pack;
  v.in = static_cast<const uint16_t*>(x);
  v.ld_in = H;
  v.out = static_cast<uint16_t*>(logits);
  v.ld_out = n_pack;
  a.op[0] = v;
  a.op[0].N = 0;
  a.table = nullptr;
  a.P = 0;
  a.E = 0;
  a.T = T;
  return launch_expert_gemm(kModePlain, kRoleRouter, 16, a, (T + 15) / 16, st);
}
}  // namespace

extern "C" {

int moe_router_logits(const void* x, int T, int H, const void* w_pack, int n_pack, void* logits,
                      void* stream) {
  CHECK_ARG(T >= 0, "T must be >= 0");
  CHECK_ARG(H >= 32 && H % 32 == 0, "hidden must be a positive multiple of 32 (got %d)", H);
  CHECK_ARG(n_pack >= 16 && n_pack % 16 == 0, "n_pack must be a positive multiple of 16 (got %d)",
            n_pack);
  CHECK_ARG(x && w_pack && logits, "null pointer");
  if (T == 0) return MOE_OK;
  hipError_t err = launch_router(x, T, H, w_pack, n_pack, logits, (hipStream_t)stream);
  if (err == hipErrorInvalidValue) return fail(MOE_EINVAL, "router: no configuration for H=%d", H);
  return hip_check(err, "router launch");
}

int moe_route_topk(const void* logits, long long ld, int T, int E, int k, long long* idx64,
                   void* w_out, int* counts, void* stream) {
  CHECK_ARG(T >= 0, "T must be >= 0");
  CHECK_ARG(E >= 1 && E <= 1024, "experts must be in [1, 1024] (got %d)", E);
  CHECK_ARG(k >= 1 && k <= 64 && k <= E, "top_k must be in [1, min(64, E)] (got %d)", k);
  CHECK_ARG(ld >= E, "logits row stride %lld < experts %d", ld, E);
  CHECK_ARG(logits && idx64 && w_out, "null pointer");
  return hip_check(launch_route(static_cast<const uint16_t*>(logits), ld, T, E, k, idx64, nullptr,
                                static_cast<uint16_t*>(w_out), counts, (hipStream_t)stream),
                   "route launch");
}

size_t moe_sort_scratch_bytes(int P, int E) { return sort_scratch_bytes(P, E); }

int moe_sort(const long long* idx64, int T, int k, int E, int bm, int has_shared, int* counts,
             int* offsets, int* order, int* table, int max_tiles, void* scratch, void* stream) {
  CHECK_ARG(T >= 0 && k >= 1 && E >= 1 && E <= 1024, "bad T/k/E (%d, %d, %d)", T, k, E);
  CHECK_ARG(bm >= 1, "bm must be >= 1");
  CHECK_ARG(max_tiles >= max_tiles_of(T, k, E, bm, has_shared), "max_tiles %d < %d", max_tiles,
            max_tiles_of(T, k, E, bm, has_shared));
  CHECK_ARG(idx64 && order && table, "null pointer");
  CHECK_ARG(sort_scratch_bytes(T * k, E) == 0 || scratch, "scratch required");
  return hip_check(launch_route_sort(nullptr, 0, nullptr, idx64, T, E, k, bm, has_shared, nullptr,
                                     nullptr, nullptr, counts, offsets, order, table, max_tiles,
                                     static_cast<int*>(scratch), (hipStream_t)stream),
                   "sort launch");
}

int moe_grouped_gate_up(const void* x, int T, int H, int E, int k, int I, const void* gate_up,
                        const float* gu_scale, int wdtype, const int* order, const int* table,
                        int max_tiles, int bm, void* act, const void* sh_gate, const void* sh_up,
                        int IS, void* act_sh, void* stream) {
  int rc = check_experts_shape(T, H, E, k, I);
  if (rc) return rc;
  CHECK_ARG(wdtype == MOE_WEIGHTS_BF16 || (wdtype == MOE_WEIGHTS_FP8_E4M3 && gu_scale),
            "bad weight dtype / missing scales");
  CHECK_ARG(x && gate_up && order && table && act, "null pointer");
  CHECK_ARG(!sh_gate || (sh_up && act_sh && IS >= 32 && IS % 32 == 0 &&
                         (((intptr_t)sh_up - (intptr_t)sh_gate) & 1) == 0),
            "shared expert needs sh_up, act_sh and IS a multiple of 32");
  if (T == 0) return MOE_OK;
  CHECK_ARG(bm == 16 || bm == 32 || bm == 64 || bm == 128 || bm == prefill_tile_rows(),
            "bm must be 16, 32, 64, 128 or %d (got %d)", prefill_tile_rows(), bm);
  return run_gate_up(x, T, H, E, k, I, gate_up, gu_scale, wdtype, sh_gate, sh_up, IS, order,
                     table, max_tiles, bm, act, act_sh, (hipStream_t)stream);
}

int moe_grouped_down(const void* act, int T, int H, int E, int k, int I, const void* down,
                     const float* dn_scale, int wdtype, const int* order, const int* table,
                     int max_tiles, int bm, void* y, const void* sh_down, int IS,
                     const void* act_sh, void* y_sh, void* stream) {
  int rc = check_experts_shape(T, H, E, k, I);
  if (rc) return rc;
  CHECK_ARG(wdtype == MOE_WEIGHTS_BF16 || (wdtype == MOE_WEIGHTS_FP8_E4M3 && dn_scale),
            "bad weight dtype / missing scales");
  CHECK_ARG(act && down && order && table && y, "null pointer");
  CHECK_ARG(!sh_down || (act_sh && y_sh && IS >= 32 && IS % 32 == 0),
            "shared expert needs act_sh, y_sh and IS a multiple of 32");
  if (T == 0) return MOE_OK;
  CHECK_ARG(bm == 16 || bm == 32 || bm == 64 || bm == 128 || bm == prefill_tile_rows(),
            "bm must be 16, 32, 64, 128 or %d (got %d)", prefill_tile_rows(), bm);
  return run_down(act, T, H, E, k, I, down, dn_scale, wdtype, sh_down, IS, act_sh, order, table,
                  max_tiles, bm, y, y_sh, (hipStream_t)stream);
}

int moe_combine(const void* y, const void* w, int T, int H, int k, const void* ysh,
                const void* seg, long long ld_seg, const void* residual, void* out, int mode,
                void* stream) {
  CHECK_ARG(T >= 0 && H % 8 == 0 && H > 0 && k >= 1, "bad combine shape");
  CHECK_ARG(mode == MOE_ROUND_PRODUCT || mode == MOE_EXACT_PRODUCT, "bad mode %d", mode);
  CHECK_ARG(!ysh || seg, "shared output needs the gate logits");
  return hip_check(launch_combine(static_cast<const uint16_t*>(y), static_cast<const uint16_t*>(w),
                                  k, static_cast<const uint16_t*>(ysh),
                                  static_cast<const uint16_t*>(seg), ld_seg,
                                  static_cast<const uint16_t*>(residual),
                                  static_cast<uint16_t*>(out), T, H, mode == MOE_ROUND_PRODUCT,
                                  (hipStream_t)stream),
                   "combine launch");
}

// ------------------------------------------------------------------------ decode stages

int moe_decode_fits(int T, int H, int E, int k, int I, int IS) {
  DecodeArgs d{};
  d.T = T, d.H = H, d.E = E, d.k = k, d.I = I, d.IS = IS;
  d.logits = reinterpret_cast<uint16_t*>(16);  // routing inside the launch
  d.sh_down = IS > 0 ? reinterpret_cast<const uint16_t*>(16) : nullptr;
  return decode_fits(d) ? 1 : 0;
}

int moe_decode_router(const void* x, int T, int H, const void* w_pack, int n_pack,
                      const void* sh_gate, const void* sh_up, int IS, void* logits, void* act_sh,
                      void* stream) {
  CHECK_ARG(x && w_pack && logits, "null pointer");
  CHECK_ARG(!sh_gate || (sh_up && act_sh), "shared gate without shared up / act_sh");
  CHECK_ARG(T >= 1 && T <= kDecMaxTokens && n_pack >= 1 &&
                (H == 512 || H == 1024 || H == 2048 || H == 4096),
            "decode router shape (T=%d H=%d n_pack=%d) not supported", T, H, n_pack);
  CHECK_ARG(!sh_gate || (IS >= 1), "bad shared intermediate %d", IS);
  DecodeArgs d{};
  d.x = static_cast<const uint16_t*>(x);
  d.T = T, d.H = H, d.IS = IS;
  d.w_pack = static_cast<const uint16_t*>(w_pack);
  d.n_pack = n_pack;
  d.sh_gate = static_cast<const uint16_t*>(sh_gate);
  d.sh_up = static_cast<const uint16_t*>(sh_up);
  d.logits = static_cast<uint16_t*>(logits);
  d.act_sh = static_cast<uint16_t*>(act_sh);
  return hip_check(launch_decode_router(d, (hipStream_t)stream), "decode router launch");
}

int moe_decode_gate_up(const void* x, int T, int H, int E, int k, int I, const void* logits,
                       int n_pack, const long long* idx64_in, const void* gate_up,
                       const float* gu_scale, int wdtype, int* idx32, void* top_k_weights,
                       long long* idx64, void* act, const void* sh_gate, const void* sh_up,
                       int IS, void* act_sh, void* stream) {
  CHECK_ARG(x && gate_up && idx32 && act, "null pointer");
  CHECK_ARG(!sh_gate || (sh_up && act_sh && IS >= 512 && IS % 512 == 0),
            "shared gate needs shared up, act_sh and IS a multiple of 512");
  CHECK_ARG(logits || idx64_in, "need logits or a given routing");
  CHECK_ARG(!logits || (top_k_weights && n_pack >= E), "routing outputs / n_pack");
  CHECK_ARG(wdtype == MOE_WEIGHTS_BF16 || (wdtype == MOE_WEIGHTS_FP8_E4M3 && gu_scale),
            "bad weight dtype / missing scales");
  DecodeArgs d{};
  d.x = static_cast<const uint16_t*>(x);
  d.T = T, d.H = H, d.E = E, d.k = k, d.I = I;
  d.gate_up = gate_up, d.gu_scale = gu_scale;
  d.fp8 = wdtype == MOE_WEIGHTS_FP8_E4M3;
  d.logits = const_cast<uint16_t*>(static_cast<const uint16_t*>(logits));
  d.n_pack = n_pack;
  d.ids_in = idx64_in;
  d.idx32 = idx32;
  d.wts = static_cast<uint16_t*>(top_k_weights);
  d.idx64 = idx64;
  d.act = static_cast<uint16_t*>(act);
  d.IS = IS;
  d.sh_gate = static_cast<const uint16_t*>(sh_gate);
  d.sh_up = static_cast<const uint16_t*>(sh_up);
  d.act_sh = static_cast<uint16_t*>(act_sh);
  d.sh_in_gate_up = sh_gate != nullptr;
  CHECK_ARG(decode_fits(d), "decode gate_up shape (T=%d H=%d E=%d k=%d I=%d) not supported", T,
            H, E, k, I);
  return hip_check(launch_decode_gate_up(d, (hipStream_t)stream), "decode gate_up launch");
}

int moe_decode_down(const void* act, int T, int H, int E, int k, int I, const int* idx32,
                    const void* top_k_weights, const void* down, const float* dn_scale,
                    int wdtype, const void* sh_down, int IS, const void* act_sh,
                    const void* logits, int n_pack, const void* residual, int mode, void* out,
                    void* stream) {
  CHECK_ARG(act && idx32 && top_k_weights && down && out, "null pointer");
  CHECK_ARG(!sh_down || (act_sh && logits && n_pack > E), "shared expert needs act_sh, logits");
  CHECK_ARG(mode == MOE_ROUND_PRODUCT || mode == MOE_EXACT_PRODUCT, "bad mode %d", mode);
  CHECK_ARG(wdtype == MOE_WEIGHTS_BF16 || (wdtype == MOE_WEIGHTS_FP8_E4M3 && dn_scale),
            "bad weight dtype / missing scales");
  DecodeArgs d{};
  d.T = T, d.H = H, d.E = E, d.k = k, d.I = I, d.IS = IS;
  d.down = down, d.dn_scale = dn_scale;
  d.fp8 = wdtype == MOE_WEIGHTS_FP8_E4M3;
  d.sh_down = static_cast<const uint16_t*>(sh_down);
  d.act_sh = const_cast<uint16_t*>(static_cast<const uint16_t*>(act_sh));
  d.logits = const_cast<uint16_t*>(static_cast<const uint16_t*>(logits));
  d.n_pack = n_pack;
  d.residual = static_cast<const uint16_t*>(residual);
  d.round_w = mode == MOE_ROUND_PRODUCT;
  d.idx32 = const_cast<int*>(idx32);
  d.wts = const_cast<uint16_t*>(static_cast<const uint16_t*>(top_k_weights));
  d.act = const_cast<uint16_t*>(static_cast<const uint16_t*>(act));
  d.out = static_cast<uint16_t*>(out);
  const uint16_t* lg = d.logits;
  d.logits = nullptr;  // the E bound of the in-launch routing does not apply here
  CHECK_ARG(decode_fits(d), "decode down shape (T=%d H=%d k=%d I=%d IS=%d) not supported", T, H,
            k, I, IS);
  d.logits = const_cast<uint16_t*>(lg);
  return hip_check(launch_decode_down(d, (hipStream_t)stream), "decode down launch");
}

// ------------------------------------------------------------------ routed experts only

namespace {
struct ExpertsWs {
  int *idx32, *counts, *offsets, *order, *table, *scratch;
  uint16_t *act, *y;
  size_t bytes;
  int MT, bm;
};
ExpertsWs carve_experts(void* base, int T, int H, int E, int k, int I, bool fp8) {
  Carver c{static_cast<char*>(base)};
  ExpertsWs w{};
  const int P = T * k;
  w.bm = tile_rows_for(T, fp8, H, I, I);
  w.MT = max_tiles_of(T, k, E, w.bm, 0);
  w.idx32 = c.take<int>(P);
  w.counts = c.take<int>(E);
  w.offsets = c.take<int>(E);
  w.order = c.take<int>(P);
  w.table = c.take<int>(3 * (size_t)w.MT + 1);
  w.scratch = c.take<int>(sort_scratch_bytes(P, E) / sizeof(int) + 1);
  w.act = c.take<uint16_t>((size_t)P * I);
  w.y = c.take<uint16_t>((size_t)P * H);
  w.bytes = c.off;
  return w;
}
}  // namespace

size_t moe_experts_workspace_bytes(int T, int H, int E, int k, int I) {
  if (T < 0 || k < 1 || E < 1) return 0;
  // the fp8 plan never needs more workspace than the bf16 one
  size_t a = carve_experts(nullptr, T, H, E, k, I, false).bytes;
  size_t b = carve_experts(nullptr, T, H, E, k, I, true).bytes;
  return a > b ? a : b;
}

int moe_experts_forward(const void* x, int T, int H, int E, int k, int I,
                        const long long* top_k_index, const void* top_k_weights,
                        const void* gate_up, const float* gu_scale, const void* down,
                        const float* dn_scale, int wdtype, int mode, void* out, void* workspace,
                        size_t workspace_bytes, void* stream) {
  int rc = check_experts_shape(T, H, E, k, I);
  if (rc) return rc;
  CHECK_ARG(mode == MOE_ROUND_PRODUCT || mode == MOE_EXACT_PRODUCT, "bad mode %d", mode);
  CHECK_ARG(wdtype == MOE_WEIGHTS_BF16 ||
                (wdtype == MOE_WEIGHTS_FP8_E4M3 && gu_scale && dn_scale),
            "bad weight dtype / missing scales");
  CHECK_ARG(x && top_k_index && top_k_weights && gate_up && down && out, "null pointer");
  if (T == 0) return MOE_OK;
  ExpertsWs w = carve_experts(workspace, T, H, E, k, I, wdtype == MOE_WEIGHTS_FP8_E4M3);
  CHECK_ARG(workspace && workspace_bytes >= w.bytes, "workspace too small: %zu < %zu",
            workspace_bytes, w.bytes);
  hipStream_t s = (hipStream_t)stream;
  if (decode_takes(T, wdtype == MOE_WEIGHTS_FP8_E4M3)) {
    DecodeArgs d{};
    d.x = static_cast<const uint16_t*>(x);
    d.T = T, d.H = H, d.E = E, d.k = k, d.I = I;
    d.gate_up = gate_up, d.gu_scale = gu_scale, d.down = down, d.dn_scale = dn_scale;
    d.fp8 = wdtype == MOE_WEIGHTS_FP8_E4M3;
    d.round_w = mode == MOE_ROUND_PRODUCT;
    d.ids_in = top_k_index;
    d.idx32 = w.idx32;
    d.wts = const_cast<uint16_t*>(static_cast<const uint16_t*>(top_k_weights));
    d.act = w.act;
    d.out = static_cast<uint16_t*>(out);
    if (decode_fits(d)) {
      HIP_TRY(launch_decode_gate_up(d, s), "decode gate_up launch");
      return hip_check(launch_decode_down(d, s), "decode down launch");
    }
  }
  HIP_TRY(launch_route_sort(nullptr, 0, nullptr, top_k_index, T, E, k, w.bm, 0, nullptr, nullptr,
                            nullptr, w.counts, w.offsets, w.order, w.table, w.MT, w.scratch, s),
          "sort launch");
  rc = run_gate_up(x, T, H, E, k, I, gate_up, gu_scale, wdtype, nullptr, nullptr, 0, w.order,
                   w.table, w.MT, w.bm, w.act, nullptr, s);
  if (rc) return rc;
  rc = run_down(w.act, T, H, E, k, I, down, dn_scale, wdtype, nullptr, 0, nullptr, w.order, w.table,
                w.MT, w.bm, w.y, nullptr, s);
  if (rc) return rc;
  return hip_check(launch_combine(w.y, static_cast<const uint16_t*>(top_k_weights), k, nullptr,
                                  nullptr, 0, nullptr, static_cast<uint16_t*>(out), T, H,
                                  mode == MOE_ROUND_PRODUCT, s),
                   "combine launch");
}

// ------------------------------------------------------------------------ whole block

namespace {
struct BlockWs {
  uint16_t* logits;
  long long* idx64;
  int* idx32;
  uint16_t* w;
  int *counts, *offsets, *order, *table, *scratch;
  uint16_t *act, *act_sh, *y, *y_sh;
  float* part;  // the router's fp32 K-quarter partial sums (router_part_takes)
  size_t bytes;
  int MT, bm;
};
BlockWs carve_block(void* base, int T, int H, int E, int k, int I, int IS, int n_pack,
                    bool fp8) {
  Carver c{static_cast<char*>(base)};
  BlockWs w{};
  const int P = T * k;
  w.bm = tile_rows_for(T, fp8, H, I, IS);
  w.MT = max_tiles_of(T, k, E, w.bm, 1);
  w.logits = c.take<uint16_t>((size_t)T * n_pack);
  w.idx64 = c.take<long long>(P);
  w.idx32 = c.take<int>(P);
  w.w = c.take<uint16_t>(P);
  w.counts = c.take<int>(E);
  w.offsets = c.take<int>(E);
  w.order = c.take<int>(P);
  w.table = c.take<int>(3 * (size_t)w.MT + 1);
  w.scratch = c.take<int>(sort_scratch_bytes(P, E) / sizeof(int) + 1);
  w.act = c.take<uint16_t>((size_t)P * I);
  w.act_sh = c.take<uint16_t>((size_t)T * IS);
  w.y = c.take<uint16_t>((size_t)P * H);
  w.y_sh = c.take<uint16_t>((size_t)T * H);
  w.part = router_part_takes(T, H, n_pack) ? c.take<float>(4 * (size_t)T * n_pack) : nullptr;
  w.bytes = c.off;
  return w;
}
}  // namespace

size_t moe_block_workspace_bytes(int T, int H, int E, int k, int I, int IS, int n_pack) {
  if (T < 0 || k < 1 || E < 1) return 0;
  size_t a = carve_block(nullptr, T, H, E, k, I, IS, n_pack, false).bytes;
  size_t b = carve_block(nullptr, T, H, E, k, I, IS, n_pack, true).bytes;
  return a > b ? a : b;
}

}  // extern "C"

namespace {

// The post-attention add + RMSNorm in front of the block (moe_block_forward_add_rms).
struct NormIn {
  const uint16_t *x, *h, *w;
  float eps;
  uint16_t *total, *out;
};

int block_forward(const void* x, int T, int H, int E, int k, int I, int IS, const void* w_pack,
                  int n_pack, const void* gate_up, const float* gu_scale, const void* down,
                  const float* dn_scale, int wdtype, const void* sh_gate, const void* sh_up,
                  const void* sh_down, const void* residual, int mode, void* out,
                  long long* top_k_index, void* top_k_weights, void* logits, void* workspace,
                  size_t workspace_bytes, void* stream, const NormIn* nm) {
  int rc = check_experts_shape(T, H, E, k, I);
  if (rc) return rc;
  CHECK_ARG(IS >= 32 && IS % 32 == 0, "shared intermediate must be a multiple of 32 (got %d)", IS);
  CHECK_ARG(n_pack >= E + 1 && n_pack % 16 == 0, "n_pack must be >= E + 1 and a multiple of 16");
  CHECK_ARG(mode == MOE_ROUND_PRODUCT || mode == MOE_EXACT_PRODUCT, "bad mode %d", mode);
  CHECK_ARG(wdtype == MOE_WEIGHTS_BF16 ||
                (wdtype == MOE_WEIGHTS_FP8_E4M3 && gu_scale && dn_scale),
            "bad weight dtype / missing scales");
  CHECK_ARG(x && w_pack && gate_up && down && sh_gate && sh_up && sh_down && out, "null pointer");
  CHECK_ARG((((intptr_t)sh_up - (intptr_t)sh_gate) & 1) == 0, "misaligned shared weights");
  if (T == 0) return MOE_OK;
  BlockWs w = carve_block(workspace, T, H, E, k, I, IS, n_pack, wdtype == MOE_WEIGHTS_FP8_E4M3);
  CHECK_ARG(workspace && workspace_bytes >= w.bytes, "workspace too small: %zu < %zu",
            workspace_bytes, w.bytes);
  hipStream_t s = (hipStream_t)stream;
  uint16_t* lg = logits ? static_cast<uint16_t*>(logits) : w.logits;
  long long* i64 = top_k_index ? top_k_index : w.idx64;
  uint16_t* wt = top_k_weights ? static_cast<uint16_t*>(top_k_weights) : w.w;
  if (decode_takes(T, wdtype == MOE_WEIGHTS_FP8_E4M3)) {
    DecodeArgs d{};
    d.x = static_cast<const uint16_t*>(x);
    d.T = T, d.H = H, d.E = E, d.k = k, d.I = I, d.IS = IS;
    d.w_pack = static_cast<const uint16_t*>(w_pack);
    d.n_pack = n_pack;
    d.gate_up = gate_up, d.gu_scale = gu_scale, d.down = down, d.dn_scale = dn_scale;
    d.fp8 = wdtype == MOE_WEIGHTS_FP8_E4M3;
    d.sh_gate = static_cast<const uint16_t*>(sh_gate);
    d.sh_up = static_cast<const uint16_t*>(sh_up);
    d.sh_down = static_cast<const uint16_t*>(sh_down);
    d.sh_in_gate_up = true;
    d.residual = static_cast<const uint16_t*>(residual);
    d.round_w = mode == MOE_ROUND_PRODUCT;
    d.logits = lg;
    d.idx64 = i64;
    d.idx32 = w.idx32;
    d.wts = wt;
    d.act = w.act;
    d.act_sh = w.act_sh;
    d.out = static_cast<uint16_t*>(out);
    if (nm) {  // the router launch normalises; gate_up reads its rows, down adds the sum
      d.norm_x = nm->x, d.norm_h = nm->h, d.norm_w = nm->w, d.norm_eps = nm->eps;
      d.norm_sum = nm->total, d.norm_out = nm->out;
      d.x = nm->out;
      d.residual = nm->h ? nm->total : nm->x;
    }
    if (decode_fits(d)) {
      HIP_TRY(launch_decode_router(d, s), "decode router launch");
      HIP_TRY(launch_decode_gate_up(d, s), "decode gate_up launch");
      return hip_check(launch_decode_down(d, s), "decode down launch");
    }
  }
  if (nm) {
    HIP_TRY(launch_add_rms(nm->x, nm->h, nm->w, T, H, nm->eps, nm->total, nm->out, s),
            "add_rms launch");
    x = nm->out;
    residual = nm->h ? nm->total : nm->x;
  }
  // The shared expert depends on x alone: where its projections would run as launches of
  // their own anyway (fp8 routed experts, prefill tiles), they run on the auxiliary stream
  // from the start of the block, beside the router and routing, and join before the combine.
  AuxStream* aux = block_side_enabled(wdtype == MOE_WEIGHTS_FP8_E4M3, w.bm) ? aux_stream(s)
                                                                               : nullptr;
  const int part = aux ? kRoutedOnly : kBoth;
  Fork fork(aux, s);  // joined before the combine, or on any early return
  if (aux) {
    HIP_TRY(fork.begin(), "fork");
    rc = run_gate_up(x, T, H, E, k, I, gate_up, gu_scale, wdtype, sh_gate, sh_up, IS, w.order,
                     w.table, w.MT, w.bm, w.act, w.act_sh, fork.aux(), kSharedOnly);
    if (rc) return rc;
    rc = run_down(w.act, T, H, E, k, I, down, dn_scale, wdtype, sh_down, IS, w.act_sh, w.order,
                  w.table, w.MT, w.bm, w.y, w.y_sh, fork.aux(), kSharedOnly);
    if (rc) return rc;
  }
  if (w.part) {
    // router partial sums, then the routing (which writes the logits), then the sort
    HIP_TRY(launch_router_part(x, T, H, w_pack, n_pack, w.part, s), "router launch");
    HIP_TRY(launch_route_part(w.part, T, n_pack, E, k, lg, i64, w.idx32, wt, s), "route launch");
    HIP_TRY(launch_route_sort(nullptr, 0, w.idx32, nullptr, T, E, k, w.bm, aux ? 0 : 1, nullptr,
                              nullptr, nullptr, w.counts, w.offsets, w.order, w.table, w.MT,
                              w.scratch, s),
            "sort launch");
  } else {
    rc = moe_router_logits(x, T, H, w_pack, n_pack, lg, stream);
    if (rc) return rc;
    HIP_TRY(launch_route_sort(lg, n_pack, nullptr, nullptr, T, E, k, w.bm, aux ? 0 : 1, i64,
                              w.idx32, wt, w.counts, w.offsets, w.order, w.table, w.MT,
                              w.scratch, s),
            "route/sort launch");
  }
  rc = run_gate_up(x, T, H, E, k, I, gate_up, gu_scale, wdtype, sh_gate, sh_up, IS, w.order,
                   w.table, w.MT, w.bm, w.act, w.act_sh, s, part);
  if (rc) return rc;
  rc = run_down(w.act, T, H, E, k, I, down, dn_scale, wdtype, sh_down, IS, w.act_sh, w.order,
                w.table, w.MT, w.bm, w.y, w.y_sh, s, part);
  if (rc) return rc;
  HIP_TRY(fork.join(), "join");
  return hip_check(launch_combine(w.y, wt, k, w.y_sh, lg + E, n_pack,
                                  static_cast<const uint16_t*>(residual),
                                  static_cast<uint16_t*>(out), T, H, mode == MOE_ROUND_PRODUCT, s),
                   "combine launch");
}

bool overlaps(const void* a, const void* b, size_t bytes) {
  const char *p = static_cast<const char*>(a), *q = static_cast<const char*>(b);
  return a && b && p < q + bytes && q < p + bytes;
}

// The aliasing and alignment rules of the add + RMSNorm entry points.
int check_norm_args(const void* x, const void* h, const void* w, int T, int H, float eps,
                    const void* total, const void* norm, const void* out) {
  CHECK_ARG(T >= 0 && H > 0 && H % 8 == 0 && H <= 512 * kAddRmsMaxChunks,
            "add_rms: H must be a positive multiple of 8 up to %d (got %d)",
            512 * kAddRmsMaxChunks, H);
  CHECK_ARG(x && w && norm && (!h || total), "add_rms: null pointer");
  CHECK_ARG(eps >= 0.f, "add_rms: eps must be >= 0 (got %g)", (double)eps);
  const size_t bytes = (size_t)T * H * 2;
  const void* ins[] = {x, h};
  const void* outs[] = {h ? total : nullptr, norm, out};
  for (const void* i : ins)
    for (const void* o : outs)
      CHECK_ARG(!overlaps(i, o, bytes), "add_rms: outputs must not overlap the inputs");
  for (int i = 0; i < 3; ++i)
    for (int j = i + 1; j < 3; ++j)
      CHECK_ARG(!overlaps(outs[i], outs[j], bytes), "add_rms: outputs must not overlap");
  CHECK_ARG(((uintptr_t)x | (uintptr_t)h | (uintptr_t)w | (uintptr_t)(h ? total : nullptr) |
             (uintptr_t)norm) % 16 == 0,
            "add_rms: rows must be 16-byte aligned");
  return MOE_OK;
}

}  // namespace

extern "C" {

int moe_block_forward(const void* x, int T, int H, int E, int k, int I, int IS,
                      const void* w_pack, int n_pack, const void* gate_up, const float* gu_scale,
                      const void* down, const float* dn_scale, int wdtype, const void* sh_gate,
                      const void* sh_up, const void* sh_down, const void* residual, int mode,
                      void* out, long long* top_k_index, void* top_k_weights, void* logits,
                      void* workspace, size_t workspace_bytes, void* stream) {
  return block_forward(x, T, H, E, k, I, IS, w_pack, n_pack, gate_up, gu_scale, down, dn_scale,
                       wdtype, sh_gate, sh_up, sh_down, residual, mode, out, top_k_index,
                       top_k_weights, logits, workspace, workspace_bytes, stream, nullptr);
}

}  // extern "C"

// ------------------------------------------------------------- no-allocation variant

namespace {

// The no-allocation entry point's workspace: a file-scope device array, one copy per GPU,
// held until the process ends. Host code never passes `scratch` itself to a kernel or a
// copy (in host code the name is a host-side stand-in, not a device address): it uses the
// address hipGetSymbolAddress gives for the current device, looked up once per device.
constexpr size_t kNoAllocScratchBytes = MOE_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

// The device address of `scratch` on the current device (looked up on the device's first
// call), or null with the error in moe_last_error().
void* scratch_ptr() {
  static std::mutex mu;
  static void* ptrs[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    fail(MOE_EHIP, "no-alloc block: no current HIP device");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      fail(MOE_EHIP, "no-alloc block: hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
      return nullptr;
    }
    ptrs[dev] = p;
  }
  return ptrs[dev];
}

}  // namespace

extern "C" {

int moe_block_forward_noalloc(const void* x, int T, int H, int E, int k, int I, int IS,
                              const void* w_pack, int n_pack, const void* gate_up,
                              const float* gu_scale, const void* down, const float* dn_scale,
                              int wdtype, const void* sh_gate, const void* sh_up,
                              const void* sh_down, const void* residual, int mode, void* out,
                              long long* top_k_index, void* top_k_weights, void* logits,
                              void* stream) {
  if (T < 0 || k < 1 || E < 1) return fail(MOE_EINVAL, "bad T/k/E (%d, %d, %d)", T, k, E);
  const size_t need = moe_block_workspace_bytes(T, H, E, k, I, IS, n_pack);
  CHECK_ARG(need <= kNoAllocScratchBytes,
            "no-alloc block: this call needs %zu bytes of workspace, more than the %zu of the "
            "static scratch (fewer tokens per call, or moe_block_forward with a workspace)",
            need, kNoAllocScratchBytes);
  if (T == 0)
    return block_forward(x, T, H, E, k, I, IS, w_pack, n_pack, gate_up, gu_scale, down,
                         dn_scale, wdtype, sh_gate, sh_up, sh_down, residual, mode, out,
                         top_k_index, top_k_weights, logits, nullptr, 0, stream, nullptr);
  void* ws = scratch_ptr();
  if (!ws) return MOE_EHIP;
  // nothing in a block workspace needs to start at zero: every kernel writes what it reads
  return block_forward(x, T, H, E, k, I, IS, w_pack, n_pack, gate_up, gu_scale, down, dn_scale,
                       wdtype, sh_gate, sh_up, sh_down, residual, mode, out, top_k_index,
                       top_k_weights, logits, ws, kNoAllocScratchBytes, stream, nullptr);
}

int moe_add_rmsnorm(const void* x, const void* h, const void* weight, int T, int H, float eps,
                    void* total, void* out, void* stream) {
  const int rc = check_norm_args(x, h, weight, T, H, eps, total, out, nullptr);
  if (rc) return rc;
  return hip_check(launch_add_rms(static_cast<const uint16_t*>(x),
                                  static_cast<const uint16_t*>(h),
                                  static_cast<const uint16_t*>(weight), T, H, eps,
                                  static_cast<uint16_t*>(total), static_cast<uint16_t*>(out),
                                  (hipStream_t)stream),
                   "add_rms launch");
}

int moe_block_forward_add_rms(const void* x, const void* h, const void* norm_weight, float eps,
                              int T, int H, int E, int k, int I, int IS, const void* w_pack,
                              int n_pack, const void* gate_up, const float* gu_scale,
                              const void* down, const float* dn_scale, int wdtype,
                              const void* sh_gate, const void* sh_up, const void* sh_down,
                              int mode, void* total, void* norm, void* out,
                              long long* top_k_index, void* top_k_weights, void* logits,
                              void* workspace, size_t workspace_bytes, void* stream) {
  const int rc = check_norm_args(x, h, norm_weight, T, H, eps, total, norm, out);
  if (rc) return rc;
  const NormIn nm{static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(h),
                  static_cast<const uint16_t*>(norm_weight), eps, static_cast<uint16_t*>(total),
                  static_cast<uint16_t*>(norm)};
  return block_forward(norm, T, H, E, k, I, IS, w_pack, n_pack, gate_up, gu_scale, down,
                       dn_scale, wdtype, sh_gate, sh_up, sh_down, nullptr, mode, out,
                       top_k_index, top_k_weights, logits, workspace, workspace_bytes, stream,
                       &nm);
}

}  // extern "C"
