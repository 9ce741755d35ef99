/* Router and whole-layer C ABI of the MI355X (gfx950) Ornith library.
 *
 * The reference computes router logits with a Triton row-dot
 * (plugin-site/ornith_g256/iu4_correctness/gates_projection.py:18-26,36-42,
 * bound via gates.py:112-121), selects experts in vLLM's topk_softmax
 * (contract plugin-site/ornith_g256/moe_base.py:53-64) and gates the shared
 * expert with rocm_unquantized_gemm + torch.sigmoid (moe_shared.py:65,
 * shared_kernel.py:101-103).  None of these has a C ABI in the reference;
 * these entries replace them with HIP kernels in a declared, fixed order:
 *   logit[t,e] = bias[e] + xor-butterfly (masks 1,2,4,8,16,32) over 64 lanes of lane partials; lane l
 *     accumulates fma(x[k], w[k], acc) for k = 8c..8c+7, c = l, l+64, l+128, l+192;
 *   p = pexp(l - max) / butterfly-sum; the 8 largest p (ties -> lower id) in
 *     descending order; weight_j = p_j / (slot-order sum of the 8 p).
 *   shared logit: the same reduction over expert_gate, rounded to bf16.
 */
#ifndef ORNITH_MI355X_MOE_H
#define ORNITH_MI355X_MOE_H
#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>
#include "ornith_routed.h"
#ifdef __cplusplus
extern "C" {
#endif

/* Replaces gates_projection.router (+ vLLM select_experts/topk_softmax, and the
 * shared-expert gate logit of moe_shared.py:65).
 *   x_bf16 [T, 2048] with row stride x_stride (elements, multiple of 8);
 *   router_w_bf16 [256, 2048]; bias_f32 [256] or NULL (a benchmark-harness
 *   additive logit term; NULL = the reference contract, moe_base.py:61);
 *   shared_gate_w_bf16 [2048] or NULL; logits_f32 [T, 257] scratch/output
 *   (column 256 = shared gate logit); topk outputs weights f32 [T,8],
 *   ids int32 [T,8]; shared_logit_bf16 [T] (written iff shared_gate_w_bf16). */
ORNITH_EXPORT hipError_t ornith_router_topk_launch(
    const void* x_bf16, int64_t x_stride, const void* router_w_bf16, const void* bias_f32,
    const void* shared_gate_w_bf16, void* logits_f32, void* topk_weights_f32, void* topk_ids_i32,
    void* shared_logit_bf16, int T, hipStream_t stream);

/* Whole quantized MoE layer: router + top-8, permutation, routed experts (A8),
 * shared expert as ninth slot (routed_storage_n32_consumer.cpp:385-401 arithmetic)
 * and the routed + shared bf16 sum done by the MoE runner.
 *   output_bf16 [T,2048] = bf16(f32(routed) + f32(shared)).
 *   topk_weights_f32 [T,8], topk_ids_i32 [T,8], shared_logit_bf16 [T] are outputs.
 * Workspace: ornith_moe_layer_get_layout(Tcap). */
ORNITH_EXPORT hipError_t ornith_moe_layer_get_layout(int Tcap, OrnithRoutedDirectLayout* out);
ORNITH_EXPORT hipError_t ornith_moe_layer_launch(
    const void* input_bf16, const void* router_w_bf16, const void* bias_f32, const void* shared_gate_w_bf16,
    const void* gate_codes, const void* gate_meta, const void* down_codes, const void* down_meta,
    const void* shared_gate_codes, const void* shared_gate_meta,
    const void* shared_down_codes, const void* shared_down_meta,
    const void* silu_f32, const void* sigmoid_bf16,
    void* workspace, size_t bytes, void* topk_weights_f32, void* topk_ids_i32, void* shared_logit_bf16,
    void* output_bf16, void* flags_u32, int T, int Tcap, hipStream_t stream);

/* The production shared expert of decode rows, fixed8
 * (plugin-site/ornith_g256/iu4_correctness/shared_kernel.py:33-62, applied by
 * shared_live.py:125-147), as one launch sequence:
 *   gu   = dense A8 G256 projection of x with the N32 gate_up bank [1024, 2048], bf16
 *          (ornith_dense_g256_launch_n32 arithmetic);
 *   act  = bf16(bf16(silu_f32[bits(gate)]) * up)   (vLLM silu_and_mul: bf16 SiLU, bf16 product);
 *   down = dense A8 projection of act with the N32 down bank [2048, 512], bf16;
 *   out  = bf16(sigmoid_bf16[bits(bf16(x . gate_w))] * down)   (scalar gate rounded to
 *          bf16, torch.sigmoid in bf16, bf16 product).
 * The reference runs it in chunks of eight rows; every row is independent, so
 * any 0 <= M <= Mcap <= 8192 is accepted.  The gate logit uses this library's
 * declared row-dot order (the router's); the reference's Triton order is not
 * pinnable.  Flags: the dense bits (1 non-finite input, 2 invalid activation,
 * 4 non-finite projection, 8 non-finite bf16).
 * Workspace: ornith_shared_fixed8_get_layout(Mcap). */
ORNITH_EXPORT hipError_t ornith_shared_fixed8_get_layout(int Mcap, size_t* workspace_bytes);
ORNITH_EXPORT hipError_t ornith_shared_fixed8_launch(
    const void* input_bf16, const void* gate_up_codes, const void* gate_up_meta,
    const void* down_codes, const void* down_meta, const void* gate_w_bf16,
    const void* silu_f32, const void* sigmoid_bf16, void* workspace, size_t bytes,
    void* output_bf16, void* flags_u32, int M, int Mcap, hipStream_t stream);

/* No reference counterpart.  For callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc): ornith_moe_layer_launch without a workspace argument.  Its
 * scratch is a static 5 MiB device array of this library (one per GPU, kept
 * until the process ends), located with hipGetSymbolAddress on the first call
 * per device.  0 <= T <= 32 (decode batches; larger T returns
 * hipErrorInvalidValue); otherwise the arguments, outputs, flags and results
 * are those of ornith_moe_layer_launch with Tcap = 32.  Nothing is allocated.
 * Every call on one GPU shares that GPU's scratch: calls that overlap in time
 * on one GPU (two streams, two threads) race and must be serialised by the
 * caller; calls in one stream are ordered and safe. */
ORNITH_EXPORT hipError_t ornith_moe_layer_launch_static(
    const void* input_bf16, const void* router_w_bf16, const void* bias_f32, const void* shared_gate_w_bf16,
    const void* gate_codes, const void* gate_meta, const void* down_codes, const void* down_meta,
    const void* shared_gate_codes, const void* shared_gate_meta,
    const void* shared_down_codes, const void* shared_down_meta,
    const void* silu_f32, const void* sigmoid_bf16,
    void* topk_weights_f32, void* topk_ids_i32, void* shared_logit_bf16,
    void* output_bf16, void* flags_u32, int T, hipStream_t stream);

/* Build identification (no reference counterpart): returns 1. */
ORNITH_EXPORT int ornith_mi355x_abi_version(void);

/* No reference counterpart.  Which kernels run a single-token (T == 1) routed
 * or whole-layer call, process-wide: 0 (default) the one-launch kernel
 * wherever its 256 blocks are resident at once on the device (else the three
 * kernels), 1 always the three kernels; -1 queries.  Returns the previous
 * setting, or -1 for another value.  Results are identical either way.  The
 * one-launch kernel raises sticky flag 64 if a block gave up waiting for
 * another block's hand-off (only possible when the grid could not be
 * resident at once, e.g. CUs taken by other work for tens of ms); see
 * ornith_mi355x_handoff_spin_limit for what that leaves in the workspace. */
ORNITH_EXPORT int ornith_mi355x_single_token_path(int path);

/* No reference counterpart.  Which kernels run the router, top-8 and sort of
 * a 2..32-token whole-layer call, process-wide: 0 (default) one launch whose
 * blocks hand logits and ids to each other, wherever its grid is resident at
 * once on the device (else three kernels), 1 always three kernels; -1
 * queries.  Returns the previous setting, or -1 for another value.  Results
 * are identical either way; the one launch raises sticky flag 64 like the
 * single-token one. */
ORNITH_EXPORT int ornith_mi355x_decode_route_path(int path);

/* No reference counterpart.  Poll rounds a one-launch kernel (single-token
 * layer, 2..32-token route) spends on one hand-off wait before it gives up
 * and raises sticky flag 64, process-wide: default 32768; 0 makes every wait
 * give up at once (for tests of the time-out path); -1 queries.  Returns the
 * previous setting, or -1 for a value outside -1..16777216.
 * A call whose arrival wait gave up (or that ran with 0) cannot confirm that
 * every block read its sequence number, so it marks the workspace poisoned:
 * every later one-launch call on that workspace gives up every wait at once,
 * raises flag 64 and computes on stale hand-off words (all indices stay in
 * range; the outputs are not meaningful) until the caller resets it. */
ORNITH_EXPORT int ornith_mi355x_handoff_spin_limit(int spins);
/* No reference counterpart.  Zeroes `bytes` of a workspace on `stream` (a fill
 * kernel, no memset node), which clears the poisoned mark above; workspace
 * NULL with bytes 0 resets the static scratch of ornith_moe_layer_launch_static
 * on the stream's device.  Workspace 256-byte aligned, bytes a multiple of 4. */
ORNITH_EXPORT hipError_t ornith_mi355x_workspace_reset(void* workspace, size_t bytes, hipStream_t stream);
/* No reference counterpart: a self-check of this library's arithmetic.  The
 * prefill gate/up epilogue computes SiLU(g) = g / (1 + portable_exp(-g)) in a
 * short form (one-step refined reciprocal, exact remainder, one correctly
 * rounded correction) when every gate value of a wave has 2^-60 <= |g| <= 80,
 * and in the full form (special cases, IEEE division) otherwise.  This call
 * evaluates both forms for every fp32 value of that domain on the device and
 * writes the number of values compared to *checked_u64 and the number whose
 * bits differ to *mismatches_u32 (device pointers; 0 mismatches expected). */
ORNITH_EXPORT hipError_t ornith_mi355x_silu_selfcheck(void* checked_u64, void* mismatches_u32, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif
