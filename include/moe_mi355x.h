/* C ABI of the MI355X (gfx950) routed-expert MoE block.
 *
 * Plain device pointers, sizes and a hipStream_t passed as void*. No entry point
 * allocates device memory or synchronises with the host: callers pass a workspace of
 * moe_*_workspace_bytes(...) bytes, so every call can be captured in a HIP graph.
 * Workspace contract: scratch only; its contents need no initialisation and are
 * meaningless between calls. Calls that share a workspace must not overlap (use one
 * workspace per stream).
 * All tensors are contiguous row-major. bf16 tensors are passed as raw 16-bit words.
 * fp8 weights are OCP e4m3fn bytes with one fp32 scale per output row.
 *
 * Return value: 0 on success; MOE_EINVAL for an unsupported shape or argument (the
 * reference's supported() predicates return False for these, engine/fast/moe_prefill.py:529-543);
 * MOE_EHIP when a launch fails. moe_last_error() gives the message of the calling
 * thread's last failure.
 *
 * Shapes: T tokens, H hidden, E experts, k experts per token, I expert intermediate,
 * IS shared-expert intermediate. Expert weights follow Transformers' Qwen3_5MoeExperts
 * (modeling_qwen3_5_moe.py:721-731): gate_up [E, 2I, H] (rows 0..I-1 gate, I..2I-1 up),
 * down [E, H, I].
 */
#ifndef MOE_MI355X_H
#define MOE_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOE_OK 0
#define MOE_EINVAL 1
#define MOE_EHIP 2

/* Weight element types. */
#define MOE_WEIGHTS_BF16 0
#define MOE_WEIGHTS_FP8_E4M3 1

/* How the routing weight multiplies an expert's bf16 output before the fp32 sum over k.
 * MOE_ROUND_PRODUCT: bf16(y * w), as Transformers' batched_mm (the decode path,
 *   engine/experts.py:99-100 -> transformers/integrations/moe.py:165-171, and
 *   engine/fast/kernels.py:163).
 * MOE_EXACT_PRODUCT: y * w exact in fp32, as the padded / sorted / grouped prefill paths
 *   (engine/experts.py:53-57,86-90; engine/fast/moe_prefill.py:580-582). */
#define MOE_ROUND_PRODUCT 1
#define MOE_EXACT_PRODUCT 2

/* Version of this interface; raised whenever an entry point's signature or contract
 * changes (2: moe_decode_gate_up takes the shared expert's rows; add + RMSNorm entry
 * points; 3: no reserved zero head in the workspaces). */
#define MOE_ABI_VERSION 3
int moe_abi_version(void);
const char* moe_last_error(void);

/* Re-read the comparison switches from the environment (MOE_DECODE=0: no decode kernels;
 * MOE_DECODE_DOWN=rows, MOE_DECODE_GU_BLOCKS=1|2|4, MOE_MIXED=0, MOE_PREFILL_SIDE=1,
 * MOE_PREFILL_SHARED_FIRST=0: alternative launch structures with the same results). The
 * library reads them once, at its first launch, and again only here, so no launch pays for
 * them. No counterpart in the reference; for tests and comparisons. Not to be called while
 * another thread launches through the library. */
void moe_reload_tuning(void);

/* Sorted rows per tile (bm) the fused entry points use for T tokens: 16 for one token,
 * 32 up to 512, above that 256 (the prefill tiles, bf16 or fp8-e4m3 weights: hidden a
 * multiple of 256, intermediates of 128) or else 64. A table passed to moe_grouped_gate_up /
 * moe_grouped_down must be built with a bm of 16, 32, 64, 128 or 256. */
int moe_tile_rows(int T);

/* Tile-table capacity for T tokens: ceil(T*k/bm) + min(E, T*k) (+ ceil(T/bm) shared tiles). */
int moe_max_tiles(int T, int k, int E, int bm, int has_shared);

/* Router logits (a1). Replaces the router F.linear of
 * modeling_qwen3_5_moe.py:768-769 / engine/fast/model.py:1159 and the packed
 * router|shared-gate GEMV of engine/fast/fused.py:745-746 + mfma.py:90-119.
 * w_pack [n_pack, H] bf16: rows 0..E-1 the router, row E the shared-expert gate
 * (shared_expert_gate.weight), the rest zero; n_pack a multiple of 16 (64 lets the
 * 64-row weight blocks of prefill-sized batches apply).
 * logits [T, n_pack] = bf16(x . w_pack^T). */
int moe_router_logits(const void* x, int T, int H, const void* w_pack, int n_pack, void* logits,
                      void* stream);

/* Softmax / top-k / renormalise (a2). Replaces prefill_kernels.route
 * (engine/fast/prefill_kernels.py:650-663, kernel :194-219) and the router of
 * modeling_qwen3_5_moe.py:770-774. Ties go to the lower expert index.
 * logits [T, ld] bf16 (first E columns used); idx64 [T, k]; w_out [T, k] bf16;
 * counts [E] int32 (optional, incremented: pass zeros). */
int moe_route_topk(const void* logits, long long ld, int T, int E, int k, long long* idx64,
                   void* w_out, int* counts, void* stream);

/* Count / stable sort / tile table (a3). Replaces the argsort + bincount of
 * engine/experts.py:71-80, moe_prefill.py:562-566 and build_tiles
 * (moe_prefill.py:509-521, _tiles_one_kernel :128-154).
 * idx64 [T, k]; counts [E], offsets [E] (exclusive cumsum), order [T*k] = stable argsort
 * of the flat ids; table [3*max_tiles + 1] in the layout of moe_prefill.py:92-126
 * (plus shared tiles (E, T*k + j*bm, T*k + T) after the routed ones when has_shared).
 * scratch: moe_sort_scratch_bytes(T*k, E) bytes. */
size_t moe_sort_scratch_bytes(int P, int E);
int moe_sort(const long long* idx64, int T, int k, int E, int bm, int has_shared, int* counts,
             int* offsets, int* order, int* table, int max_tiles, void* scratch, void* stream);

/* Grouped expert gate_up (a4 / a8): act[r] = bf16(bf16(silu(bf16 g)) * bf16 u) for sorted
 * row r of pair order[r] (token order[r] / k). Replaces moe_prefill._gate_up_kernel
 * (engine/fast/moe_prefill.py:156-211) and kernels._moe_gate_up_kernel (kernels.py:88-125).
 * act [T*k, I] bf16. gu_scale [E, 2I] fp32 for fp8 weights, else null.
 * With sh_gate / sh_up [IS, H] (and a table built with has_shared) the same launch also
 * computes the shared expert's act_sh [T, IS] (a6; prefill_kernels.py:232-251). */
int moe_grouped_gate_up(const void* x, int T, int H, int E, int k, int I, const void* gate_up,
                        const float* gu_scale, int wdtype, const int* order, const int* table,
                        int max_tiles, int bm, void* act, const void* sh_gate, const void* sh_up,
                        int IS, void* act_sh, void* stream);

/* Grouped expert down (a5 / a9): y[order[r]] = bf16(act[r] . Wd[e]) at each pair's own row.
 * Replaces moe_prefill._down_kernel / _down_stream_kernel (moe_prefill.py:212-319).
 * y [T*k, H] bf16. dn_scale [E, H] fp32 for fp8 weights, else null.
 * With sh_down [H, IS] the same launch also writes y_sh [T, H] = bf16(act_sh . Wsd). */
int moe_grouped_down(const void* act, int T, int H, int E, int k, int I, const void* down,
                     const float* dn_scale, int wdtype, const int* order, const int* table,
                     int max_tiles, int bm, void* y, const void* sh_down, int IS,
                     const void* act_sh, void* y_sh, void* stream);

/* Combine (a7 / a10): out[t] = bf16(bf16(sum_j term(y[t*k+j], w[t,j]))
 *   + bf16(bf16(sigmoid(seg[t])) * ysh[t])) (+ residual). Replaces
 * prefill_kernels._moe_combine_kernel (engine/fast/prefill_kernels.py:253-273) and the
 * weighted sums of transformers/integrations/moe.py:165-174 / engine/experts.py:53-57.
 * ysh / seg / residual may be null. mode: MOE_ROUND_PRODUCT or MOE_EXACT_PRODUCT. */
int moe_combine(const void* y, const void* w, int T, int H, int k, const void* ysh,
                const void* seg, long long ld_seg, const void* residual, void* out, int mode,
                void* stream);

/* Decode stages (T <= 4 tokens; H 512, 1024, 2048 or 4096, I and IS 512 or 1024,
 * E <= 512, T*k <= 64): the three launches of engine/fast/fused.py's FusedDecode._moe
 * (fused.py:887-932). moe_decode_fits says whether a shape fits this path; the fused
 * entry points below take it on their own for such shapes, with bf16 or fp8-e4m3 experts
 * (MOE_DECODE=0 turns the decode path off). */
int moe_decode_fits(int T, int H, int E, int k, int I, int IS);

/* Stage 1: router logits [T, n_pack] (as moe_router_logits) and, with sh_gate / sh_up
 * [IS, H], act_sh [T, IS] = bf16(bf16(silu(bf16 g)) * bf16 u) of the shared expert in the
 * same launch. Replaces the packed router|shared GEMV of fused.py:745-746 / 798-840. */
int moe_decode_router(const void* x, int T, int H, const void* w_pack, int n_pack,
                      const void* sh_gate, const void* sh_up, int IS, void* logits, void* act_sh,
                      void* stream);

/* Stage 2: act [T*k, I] = SwiGLU of the routed experts. With logits (first E columns, row
 * stride n_pack) the softmax / top-k runs inside the launch and the routing is written to
 * idx32 [T, k], top_k_weights [T, k] bf16 and idx64 [T, k] (optional); without, idx64_in
 * gives it and idx32 receives a copy. With sh_gate / sh_up ([IS, H], IS a multiple of 512)
 * the same launch also writes act_sh [T, IS] (then stage 1 is called without them; the bits
 * are the same either way). Replaces _topk (fused.py:554-570) and _moe_up_kernel with
 * FUSE_TOPK (fused.py:582-632). */
int moe_decode_gate_up(const void* x, int T, int H, int E, int k, int I, const void* logits,
                       int n_pack, const long long* idx64_in, const void* gate_up,
                       const float* gu_scale, int wdtype, int* idx32, void* top_k_weights,
                       long long* idx64, void* act, const void* sh_gate, const void* sh_up,
                       int IS, void* act_sh, void* stream);

/* Stage 3: out [T, H] = bf16(bf16(sum_j term_j) + bf16(bf16(sigmoid(seg)) * y_sh))
 * (+ residual), term_j = bf16(w_j * bf16(act_p . Wd[e_p])) under MOE_ROUND_PRODUCT, with
 * y_sh = bf16(act_sh . Wsd) and seg = logits[t, E]. sh_down null: routed experts only (no
 * shared term; logits unused). Replaces _moe_down_kernel (fused.py:635-692). */
int moe_decode_down(const void* act, int T, int H, int E, int k, int I, const int* idx32,
                    const void* top_k_weights, const void* down, const float* dn_scale,
                    int wdtype, const void* sh_down, int IS, const void* act_sh,
                    const void* logits, int n_pack, const void* residual, int mode, void* out,
                    void* stream);

/* Routed experts only (surface 1): the experts_forward(self, hidden_states, top_k_index,
 * top_k_weights) of engine/experts.py:93-102 (batched_mm for T <= 16, padded bmm above).
 * out [T, H] bf16. */
size_t moe_experts_workspace_bytes(int T, int H, int E, int k, int I);
int moe_experts_forward(const void* x, int T, int H, int E, int k, int I,
                        const long long* top_k_index, const void* top_k_weights,
                        const void* gate_up, const float* gu_scale, const void* down,
                        const float* dn_scale, int wdtype, int mode, void* out, void* workspace,
                        size_t workspace_bytes, void* stream);

/* Whole block (surface 2): router + top-k + routed experts + gated shared expert
 * (+ residual). Replaces FastModel._moe (engine/fast/model.py:1139-1179),
 * prefill_kernels.moe (prefill_kernels.py:676-742), FusedDecode._moe (fused.py:887-932)
 * and Qwen3_5MoeSparseMoeBlock.forward (modeling_qwen3_5_moe.py:787-800).
 * sh_gate / sh_up [IS, H], sh_down [H, IS] bf16. residual [T, H] or null.
 * top_k_index [T, k] int64 / top_k_weights [T, k] bf16 / logits [T, n_pack] bf16 are
 * optional outputs (null: kept in the workspace). */
size_t moe_block_workspace_bytes(int T, int H, int E, int k, int I, int IS, int n_pack);
int moe_block_forward(const void* x, int T, int H, int E, int k, int I, int IS,
                      const void* w_pack, int n_pack, const void* gate_up, const float* gu_scale,
                      const void* down, const float* dn_scale, int wdtype, const void* sh_gate,
                      const void* sh_up, const void* sh_down, const void* residual, int mode,
                      void* out, long long* top_k_index, void* top_k_weights, void* logits,
                      void* workspace, size_t workspace_bytes, void* stream);

/* Whole block without a caller workspace (no counterpart in the reference): for callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Same arguments and results as moe_block_forward, minus
 * workspace / workspace_bytes: the workspace is a static device array of
 * MOE_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends, whose address is looked
 * up on the first call on each device. Calls whose moe_block_workspace_bytes(...) exceeds
 * it fail with MOE_EINVAL (at the full Qwen3.6 layer shape: up to ~350 tokens). No call
 * allocates or frees anything. Every call on one GPU uses that GPU's one array: calls that
 * overlap on one GPU (two streams, two threads) race and must be serialised by the caller. */
#define MOE_NOALLOC_SCRATCH_BYTES (16u << 20)
int moe_block_forward_noalloc(const void* x, int T, int H, int E, int k, int I, int IS,
                              const void* w_pack, int n_pack, const void* gate_up,
                              const float* gu_scale, const void* down, const float* dn_scale,
                              int wdtype, const void* sh_gate, const void* sh_up,
                              const void* sh_down, const void* residual, int mode, void* out,
                              long long* top_k_index, void* top_k_weights, void* logits,
                              void* stream);

/* Post-attention residual add + zero-centred RMSNorm: total = bf16(x + h) and
 * out = bf16(total * rsqrt(mean(total^2) + eps) * (1 + weight)), fp32 in between; h null:
 * no add (total is not written, the norm is of x). x, h, total, out [T, H] bf16 with
 * 16-byte-aligned rows, weight [H] bf16, H a multiple of 8 up to 8192; outputs must not
 * overlap the inputs. Replaces kernels.add_rms (engine/fast/kernels.py:636-650, math of
 * _add_rms_kernel kernels.py:507-523, as Transformers' Qwen3_5MoeRMSNorm
 * modeling_qwen3_5_moe.py:801-815). */
int moe_add_rmsnorm(const void* x, const void* h, const void* weight, int T, int H, float eps,
                    void* total, void* out, void* stream);

/* The post-attention add_rms and the MoE block of one decoder layer:
 * (total, norm) = add_rms(x, h, norm_weight, eps), out = total + MoE(norm) (h null: x stands
 * for total). Replaces `x, h = kernels.add_rms(x, h, post_attention_layernorm.weight, eps)`
 * followed by the block with x as residual (engine/fast/model.py:888-891; fused.py:1074-1076
 * with FusedDecode._moe fused.py:887-932). total and norm are written too. On the decode path
 * the norm runs inside the router launch (no launch of its own); elsewhere one add_rms launch
 * precedes the block. Other arguments, the workspace (moe_block_workspace_bytes) and the
 * optional routing outputs are those of moe_block_forward. */
int moe_block_forward_add_rms(const void* x, const void* h, const void* norm_weight, float eps,
                              int T, int H, int E, int k, int I, int IS, const void* w_pack,
                              int n_pack, const void* gate_up, const float* gu_scale,
                              const void* down, const float* dn_scale, int wdtype,
                              const void* sh_gate, const void* sh_up, const void* sh_down,
                              int mode, void* total, void* norm, void* out,
                              long long* top_k_index, void* top_k_weights, void* logits,
                              void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOE_MI355X_H */
