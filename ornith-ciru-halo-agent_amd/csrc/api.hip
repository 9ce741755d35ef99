// extern "C" entry points.  Argument validation is host-only and runs before
// any launch; every entry enqueues on the caller's stream and allocates
// nothing.  The references for each entry are in include/ornith_*.h.
#include <algorithm>
#include <mutex>
#include "kernels.hpp"
#include "timing.hpp"
#include "decode.hpp"
#include "validate.hpp"
#include "../../include/ornith_routed.h"
#include "../../include/ornith_dense.h"
#include "../../include/ornith_moe.h"
#include "../../include/ornith_timing.h"

using namespace ornith;

namespace {

#define TRY(expr) do { hipError_t _s = (expr); if (_s != hipSuccess) return _s; } while (0)

constexpr int kMaxTokens = 8192;
constexpr int kGateN = 2 * kInter, kDownN = kHidden;

// Workspace plan shared by the routed, shared-slot and whole-layer entries.
struct RoutedPlan {
    OrnithRoutedDirectLayout l;
    size_t permute, logits, router_split, decode;
};

RoutedPlan routed_plan(int Tcap, bool shared_slot, bool layer) {
    RoutedPlan p{};
    size_t cursor = 0;
    const size_t t = size_t(Tcap), rs = t * kTop + (shared_slot ? t : 0);
    auto add = [&](size_t& field, size_t bytes) { field = cursor; cursor = align256(cursor + bytes); };
    add(p.l.gate_x, 0);
    add(p.l.gate_low, t * kHidden);                       // int8 activation words
    add(p.l.gate_high, 0);
    add(p.l.gate_scales, t * (kHidden / kGroup) * 2);
    add(p.l.gate_sums, t * (kHidden / kGroup) * 4);
    add(p.l.gate_y, rs * kGateN * 4);
    add(p.l.middle, rs * kInter * 4);
    add(p.l.down_x, 0);
    add(p.l.down_low, rs * kInter);                       // int8 activation words
    add(p.l.down_high, 0);
    add(p.l.down_scales, rs * (kInter / kGroup) * 2);
    add(p.l.down_sums, rs * (kInter / kGroup) * 4);
    add(p.l.route_out, rs * kHidden * 4);
    add(p.l.final_f32, t * kHidden * 4);
    add(p.permute, permute_scratch_bytes(int(t * kTop), shared_slot ? int(t) : 0));
    if (layer) add(p.logits, t * kLogitStride * 4);
    if (layer) add(p.router_split, router_split_bytes(Tcap));
    add(p.decode, decode_scratch_bytes());
    p.l.workspace_bytes = cursor;
    return p;
}

// Prefill path (T > 32): permutation into expert segments and 64-route
// tiles, int8-MFMA grouped projections, middle quantisation, slot reduce.
hipError_t run_routed(const RoutedPlan& p, void* ws, const void* input, const float* weights, const int32_t* ids,
                      const void* gate_codes, const void* gate_meta, const void* down_codes, const void* down_meta,
                      const void* sg_codes, const void* sg_meta, const void* sd_codes, const void* sd_meta,
                      const uint16_t* shared_logit, const float* silu, const uint16_t* sigmoid, int qmax,
                      uint16_t* out, uint16_t* shared_out, uint16_t* layer_out, uint32_t* sticky, int T, int Tcap,
                      hipStream_t s, bool counted = false) {
    const bool shared = sg_codes != nullptr;
    const int R = T * kTop, RS = R + (shared ? T : 0);
    const PermuteScratch ps = carve_permute(at<void>(ws, p.permute), Tcap * kTop, shared ? Tcap : 0);
    auto gw = at<uint32_t>(ws, p.l.gate_low);
    auto gs = at<uint16_t>(ws, p.l.gate_scales);
    auto gsum = at<int32_t>(ws, p.l.gate_sums);
    // the A8 gate input rides on the bank-scan launch (the A4 one has its own)
    const ActJob act{static_cast<const uint16_t*>(input), T, shared ? nullptr : ids, gw, gs, gsum};
    TRY(launch_permute(ids, R, T, shared, ps, sticky, 64, s, counted, qmax == 127 ? &act : nullptr));
    if (qmax != 127)
        TRY(launch_act_bf16(static_cast<const uint16_t*>(input), kHidden, T, kHidden, qmax, shared ? nullptr : ids, gw,
                            gs, gsum, sticky, kFlagNonfiniteInput, kFlagInvalidActivation, s));
    const int max_tiles = (RS + 63) / 64 + (R < kExperts ? R : kExperts) + (shared ? 1 : 0);
    MfmaArgs a{};
    a.segments = ps.segments;
    a.tiles = ps.tiles;
    a.ntiles = ps.meta + 1;
    a.routes = ps.routes;
    a.R = R;
    a.codes = static_cast<const uint32_t*>(gate_codes);
    a.meta = static_cast<const uint32_t*>(gate_meta);
    a.shared_codes = static_cast<const uint32_t*>(sg_codes);
    a.shared_meta = static_cast<const uint32_t*>(sg_meta);
    a.bank_words = kGateBankWords;
    a.bank_meta_words = kGateBankMeta;
    a.act_words = gw; a.act_scales = gs; a.act_sums = gsum;
    a.K = kHidden;
    a.out = at<float>(ws, p.l.middle);
    a.silu_table = silu;
    a.sticky = sticky;
    // above 2048 tokens nearly every tile is full: keep each tile on one XCD
    a.tile_xcd = T > 2048 ? 1 : 0;
    TRY(launch_grouped_mfma(a, true, max_tiles, s));
    auto dw = at<uint32_t>(ws, p.l.down_low);
    auto dsc = at<uint16_t>(ws, p.l.down_scales);
    auto dsum = at<int32_t>(ws, p.l.down_sums);
    // middle rows are in permuted route order; offsets[257] = routes with a valid bank
    TRY(launch_quant_middle_permuted(at<float>(ws, p.l.middle), RS, ps.offsets + kExperts + 1, qmax, dw, dsc, dsum,
                                     sticky, s));
    a.codes = static_cast<const uint32_t*>(down_codes);
    a.meta = static_cast<const uint32_t*>(down_meta);
    a.shared_codes = static_cast<const uint32_t*>(sd_codes);
    a.shared_meta = static_cast<const uint32_t*>(sd_meta);
    a.bank_words = kDownBankWords;
    a.bank_meta_words = kDownBankMeta;
    a.act_words = dw; a.act_scales = dsc; a.act_sums = dsum;
    a.K = kInter;
    // down: an XCD's m-tiles contiguous up to 2048 tokens (block orders: proj_mfma.hip)
    a.tile_xcd = T > 2048 ? 0 : 2;
    a.out = at<float>(ws, p.l.route_out);
    TRY(launch_grouped_mfma(a, false, max_tiles, s));
    return launch_reduce(at<float>(ws, p.l.route_out), weights, ids, T, out ? at<float>(ws, p.l.final_f32) : nullptr,
                         out, shared_logit, shared ? sigmoid : nullptr, shared_out, layer_out, sticky, s);
}

// Decode path (T <= 32): three kernels, see decode.hip.
hipError_t run_decode(const RoutedPlan& p, void* ws, const void* input, const float* weights, const int32_t* ids,
                      const void* gate_codes, const void* gate_meta, const void* down_codes, const void* down_meta,
                      const void* sg_codes, const void* sg_meta, const void* sd_codes, const void* sd_meta,
                      uint16_t* shared_logit, const float* silu, const uint16_t* sigmoid, int qmax, uint16_t* out,
                      uint16_t* shared_out, uint16_t* layer_out, uint32_t* sticky, int T, hipStream_t s,
                      const void* router_w = nullptr, const void* bias = nullptr, const void* shared_gate_w = nullptr,
                      float* topk_w = nullptr, int32_t* topk_ids = nullptr) {
    DecodeArgs a{};
    a.T = T;
    a.x = static_cast<const uint16_t*>(input);
    a.router_w = static_cast<const uint16_t*>(router_w);
    a.bias = static_cast<const float*>(bias);
    a.shared_gate_w = static_cast<const uint16_t*>(shared_gate_w);
    a.topk_w = topk_w;
    a.topk_ids = topk_ids;
    a.ids_in = ids;
    a.reduce_w = router_w ? topk_w : weights;
    a.reduce_ids = router_w ? topk_ids : ids;
    a.w13_codes = static_cast<const uint32_t*>(gate_codes);
    a.w13_meta = static_cast<const uint32_t*>(gate_meta);
    a.w2_codes = static_cast<const uint32_t*>(down_codes);
    a.w2_meta = static_cast<const uint32_t*>(down_meta);
    a.s13_codes = static_cast<const uint32_t*>(sg_codes);
    a.s13_meta = static_cast<const uint32_t*>(sg_meta);
    a.s2_codes = static_cast<const uint32_t*>(sd_codes);
    a.s2_meta = static_cast<const uint32_t*>(sd_meta);
    a.silu_table = silu;
    a.sigmoid_table = sigmoid;
    a.shared_logit = shared_logit;
    a.x_words = at<uint32_t>(ws, p.l.gate_low);
    a.x_scales = at<uint16_t>(ws, p.l.gate_scales);
    a.x_sums = at<int32_t>(ws, p.l.gate_sums);
    a.middle = at<float>(ws, p.l.middle);
    a.route_out = at<float>(ws, p.l.route_out);
    carve_decode(at<void>(ws, p.decode), a);
    a.final_f32 = out ? at<float>(ws, p.l.final_f32) : nullptr;
    a.out = out;
    a.shared_out = shared_out;
    a.layer_out = layer_out;
    a.sticky = sticky;
    return launch_decode(a, router_w != nullptr, sg_codes != nullptr, qmax, s);
}

template <int QMAX>
hipError_t routed_launch(const void* input, const void* weights, const void* ids, const void* gate_codes,
                         const void* gate_meta, const void* down_codes, const void* down_meta, void* workspace,
                         size_t bytes, void* output, void* flags, int T, int Tcap, hipStream_t stream) {
    if (Tcap < 0 || Tcap > kMaxTokens || T < 0 || T > Tcap) return hipErrorInvalidValue;
    const RoutedPlan p = routed_plan(Tcap, false, false);
    if (bytes < p.l.workspace_bytes) return hipErrorInvalidValue;
    if (!T) return hipSuccess;
    if (!input || !weights || !ids || !gate_codes || !gate_meta || !down_codes || !down_meta || !workspace || !output ||
        !flags)
        return hipErrorInvalidValue;
    if (!aligned(input, 16) || !aligned(weights, 4) || !aligned(ids, 4) || !aligned(gate_codes, 16) ||
        !aligned(down_codes, 16) || !aligned(gate_meta, 4) || !aligned(down_meta, 4) || !aligned(workspace, 256) ||
        !aligned(output, 8) || !aligned(flags, 4))
        return hipErrorInvalidValue;
    if (T <= kDecodeMaxTokens)
        return run_decode(p, workspace, input, static_cast<const float*>(weights), static_cast<const int32_t*>(ids),
                          gate_codes, gate_meta, down_codes, down_meta, nullptr, nullptr, nullptr, nullptr, nullptr,
                          nullptr, nullptr, QMAX, static_cast<uint16_t*>(output), nullptr, nullptr,
                          static_cast<uint32_t*>(flags), T, stream);
    return run_routed(p, workspace, input, static_cast<const float*>(weights), static_cast<const int32_t*>(ids),
                      gate_codes, gate_meta, down_codes, down_meta, nullptr, nullptr, nullptr, nullptr, nullptr,
                      nullptr, nullptr, QMAX, static_cast<uint16_t*>(output), nullptr, nullptr,
                      static_cast<uint32_t*>(flags), T, Tcap, stream);
}

// ---- dense helpers --------------------------------------------------------------
bool dense_shape(int N, int K) {
    return N > 0 && (N <= 12288 || N == 248320) && N % 16 == 0 && K > 0 && K <= 8192 && K % kGroup == 0;
}

OrnithDenseG256Layout dense_layout(int Mcap, int N, int K) {
    OrnithDenseG256Layout l{};
    size_t cursor = 0;
    const size_t m = size_t(Mcap);
    auto add = [&](size_t& field, size_t bytes) { field = cursor; cursor = align256(cursor + bytes); };
    add(l.transformed, 0);
    add(l.low, m * K);                       // int8 activation words
    add(l.high, 0);
    add(l.scales, m * (K / kGroup) * 2);
    add(l.sums, m * (K / kGroup) * 4);
    add(l.projection, m * N * 4);
    l.workspace_bytes = cursor;
    return l;
}

hipError_t dense_run(const void* input, const void* codes, const void* meta, void* ws, const OrnithDenseG256Layout& l,
                     float* projection, uint16_t* out, uint32_t* sticky, int M, int N, int K, int tile, hipStream_t s) {
    auto w = at<uint32_t>(ws, l.low);
    auto sc = at<uint16_t>(ws, l.scales);
    auto su = at<int32_t>(ws, l.sums);
    ProjArgs a{};
    if (M <= kDenseFusedRows) {
        // the projection prepares its own activations
        a.dense_x = static_cast<const uint16_t*>(input);
        a.flag_input = kDenseNonfiniteInput;
        a.flag_act = kDenseInvalidActivation;
    } else {
        TRY(launch_act_bf16(static_cast<const uint16_t*>(input), K, M, K, 127, nullptr, w, sc, su, sticky,
                            kDenseNonfiniteInput, kDenseInvalidActivation, s));
    }
    a.codes = static_cast<const uint32_t*>(codes);
    a.meta = static_cast<const uint32_t*>(meta);
    a.dense_rows = M;
    a.act_words = w; a.act_scales = sc; a.act_sums = su;
    a.out = projection; a.out_bf16 = out;
    a.N = N; a.K = K; a.tile = tile;
    a.sticky = sticky; a.flag_projection = kDenseNonfiniteProjection; a.flag_bf16 = kDenseNonfiniteBf16;
    return launch_project_gemv(a, 1, Out::Dense, s);
}

}  // namespace

// =============================================================================
// Routed
// =============================================================================
extern "C" hipError_t ornith_routed_direct_get_layout(int Tcap, OrnithRoutedDirectLayout* out) {
    if (!out || Tcap < 0 || Tcap > kMaxTokens) return hipErrorInvalidValue;
    *out = routed_plan(Tcap, false, false).l;
    return hipSuccess;
}

extern "C" hipError_t ornith_routed_direct_launch(const void* input, const void* weights, const void* ids,
                                                  const void* gate_codes, const void* gate_meta, const void* down_codes,
                                                  const void* down_meta, void* workspace, size_t bytes, void* output,
                                                  void* flags, int T, int Tcap, hipStream_t stream) {
    return routed_launch<127>(input, weights, ids, gate_codes, gate_meta, down_codes, down_meta, workspace, bytes,
                              output, flags, T, Tcap, stream);
}

extern "C" hipError_t ornith_routed_direct_launch_a4(const void* input, const void* weights, const void* ids,
                                                     const void* gate_codes, const void* gate_meta,
                                                     const void* down_codes, const void* down_meta, void* workspace,
                                                     size_t bytes, void* output, void* flags, int T, int Tcap,
                                                     hipStream_t stream) {
    return routed_launch<7>(input, weights, ids, gate_codes, gate_meta, down_codes, down_meta, workspace, bytes, output,
                            flags, T, Tcap, stream);
}

extern "C" hipError_t ornith_routed_direct_launch_a4_prefill(const void* input, const void* weights, const void* ids,
                                                             const void* gate_codes, const void* gate_meta,
                                                             const void* down_codes, const void* down_meta,
                                                             void* workspace, size_t bytes, void* output, void* flags,
                                                             int T, int Tcap, hipStream_t stream) {
    if (T > 64)
        return routed_launch<7>(input, weights, ids, gate_codes, gate_meta, down_codes, down_meta, workspace, bytes,
                                output, flags, T, Tcap, stream);
    return routed_launch<127>(input, weights, ids, gate_codes, gate_meta, down_codes, down_meta, workspace, bytes,
                              output, flags, T, Tcap, stream);
}

// 32 in the N32-storage build, 16 in the N16 build (the bank tile the routed entries read)
extern "C" int ornith_routed_storage_n32(void) { return kRoutedTile; }
extern "C" int ornith_routed_prefill_output_tile(void) { return 32; }

extern "C" hipError_t ornith_routed_shared_get_layout(int Tcap, OrnithRoutedDirectLayout* out) {
    if (!out || Tcap < 0 || Tcap > 16) return hipErrorInvalidValue;
    *out = routed_plan(Tcap, true, false).l;
    return hipSuccess;
}

extern "C" hipError_t ornith_routed_direct_launch_shared_tables(
    const void* input, const void* weights, const void* ids, const void* gate_codes, const void* gate_meta,
    const void* down_codes, const void* down_meta, const void* shared_gate_codes, const void* shared_gate_meta,
    const void* shared_down_codes, const void* shared_down_meta, const void* shared_logit, const void* shared_silu,
    const void* shared_sigmoid, void* workspace, size_t bytes, void* output, void* shared_output, void* flags, int T,
    int Tcap, hipStream_t stream) {
    if (Tcap < 0 || Tcap > 16 || T < 0 || T > Tcap) return hipErrorInvalidValue;
    const RoutedPlan p = routed_plan(Tcap, true, false);
    if (bytes < p.l.workspace_bytes) return hipErrorInvalidValue;
    if (!T) return hipSuccess;
    const void* req[] = {input, weights, ids, gate_codes, gate_meta, down_codes, down_meta, shared_gate_codes,
                         shared_gate_meta, shared_down_codes, shared_down_meta, shared_logit, shared_silu,
                         shared_sigmoid, workspace, output, shared_output, flags};
    for (const void* q : req) if (!q) return hipErrorInvalidValue;
    if (!aligned(input, 16) || !aligned(gate_codes, 16) || !aligned(down_codes, 16) || !aligned(shared_gate_codes, 16) ||
        !aligned(shared_down_codes, 16) || !aligned(workspace, 256) || !aligned(output, 8) ||
        !aligned(shared_output, 8) || !aligned(flags, 4))
        return hipErrorInvalidValue;
    return run_decode(p, workspace, input, static_cast<const float*>(weights), static_cast<const int32_t*>(ids),
                      gate_codes, gate_meta, down_codes, down_meta, shared_gate_codes, shared_gate_meta,
                      shared_down_codes, shared_down_meta, static_cast<uint16_t*>(const_cast<void*>(shared_logit)),
                      static_cast<const float*>(shared_silu), static_cast<const uint16_t*>(shared_sigmoid), 127,
                      static_cast<uint16_t*>(output), static_cast<uint16_t*>(shared_output), nullptr,
                      static_cast<uint32_t*>(flags), T, stream);
}

// =============================================================================
// Router and whole layer
// =============================================================================
extern "C" hipError_t ornith_router_topk_launch(const void* x, int64_t x_stride, const void* router_w,
                                                const void* bias, const void* shared_gate_w, void* logits,
                                                void* topk_weights, void* topk_ids, void* shared_logit, int T,
                                                hipStream_t stream) {
    if (T < 0 || T > kMaxTokens || x_stride < kHidden || x_stride % 8) return hipErrorInvalidValue;
    if (!T) return hipSuccess;
    if (!x || !router_w || !logits || !topk_weights || !topk_ids || (shared_gate_w && !shared_logit))
        return hipErrorInvalidValue;
    if (!aligned(x, 16) || !aligned(router_w, 16) || (shared_gate_w && !aligned(shared_gate_w, 16)) ||
        !aligned(logits, 4) || !aligned(topk_weights, 4) || !aligned(topk_ids, 4))
        return hipErrorInvalidValue;
    auto lg = static_cast<float*>(logits);
    TRY(launch_router(static_cast<const uint16_t*>(x), x_stride, T, static_cast<const uint16_t*>(router_w),
                      static_cast<const uint16_t*>(shared_gate_w), static_cast<const float*>(bias), lg, kLogitStride,
                      stream));
    return launch_topk(lg, kLogitStride, T, static_cast<float*>(topk_weights), static_cast<int32_t*>(topk_ids),
                       shared_gate_w ? lg + kExperts : nullptr, kLogitStride,
                       shared_gate_w ? static_cast<uint16_t*>(shared_logit) : nullptr, stream);
}

extern "C" hipError_t ornith_moe_layer_get_layout(int Tcap, OrnithRoutedDirectLayout* out) {
    if (!out || Tcap < 0 || Tcap > kMaxTokens) return hipErrorInvalidValue;
    *out = routed_plan(Tcap, true, true).l;
    return hipSuccess;
}

extern "C" hipError_t ornith_moe_layer_launch(
    const void* input, const void* router_w, const void* bias, const void* shared_gate_w, const void* gate_codes,
    const void* gate_meta, const void* down_codes, const void* down_meta, const void* shared_gate_codes,
    const void* shared_gate_meta, const void* shared_down_codes, const void* shared_down_meta, const void* silu,
    const void* sigmoid, void* workspace, size_t bytes, void* topk_weights, void* topk_ids, void* shared_logit,
    void* output, void* flags, int T, int Tcap, hipStream_t stream) {
    if (Tcap < 0 || Tcap > kMaxTokens || T < 0 || T > Tcap) return hipErrorInvalidValue;
    const RoutedPlan p = routed_plan(Tcap, true, true);
    if (bytes < p.l.workspace_bytes) return hipErrorInvalidValue;
    if (!T) return hipSuccess;
    const void* req[] = {input, router_w, shared_gate_w, gate_codes, gate_meta, down_codes, down_meta,
                         shared_gate_codes, shared_gate_meta, shared_down_codes, shared_down_meta, silu, sigmoid,
                         workspace, topk_weights, topk_ids, shared_logit, output, flags};
    for (const void* q : req) if (!q) return hipErrorInvalidValue;
    if (!aligned(input, 16) || !aligned(router_w, 16) || !aligned(shared_gate_w, 16) || !aligned(gate_codes, 16) ||
        !aligned(down_codes, 16) || !aligned(shared_gate_codes, 16) || !aligned(shared_down_codes, 16) ||
        !aligned(workspace, 256) || !aligned(output, 8) || !aligned(flags, 4))
        return hipErrorInvalidValue;
    if (T <= kDecodeMaxTokens)
        return run_decode(p, workspace, input, nullptr, nullptr, gate_codes, gate_meta, down_codes, down_meta,
                          shared_gate_codes, shared_gate_meta, shared_down_codes, shared_down_meta,
                          static_cast<uint16_t*>(shared_logit), static_cast<const float*>(silu),
                          static_cast<const uint16_t*>(sigmoid), 127, nullptr, nullptr, static_cast<uint16_t*>(output),
                          static_cast<uint32_t*>(flags), T, stream, router_w, bias, shared_gate_w,
                          static_cast<float*>(topk_weights), static_cast<int32_t*>(topk_ids));
    auto logits = at<float>(workspace, p.logits);
    // the last token groups' logits may be completed by the top-k launch
    float* split = router_split_groups(T) ? at<float>(workspace, p.router_split) : nullptr;
    // top-8 also counts the routed banks per 16-token block (permutation step 1)
    const PermuteScratch ps = carve_permute(at<void>(workspace, p.permute), Tcap * kTop, Tcap);
    TRY(launch_router(static_cast<const uint16_t*>(input), kHidden, T, static_cast<const uint16_t*>(router_w),
                      static_cast<const uint16_t*>(shared_gate_w), static_cast<const float*>(bias), logits,
                      kLogitStride, stream, split));
    TRY(launch_topk(logits, kLogitStride, T, static_cast<float*>(topk_weights), static_cast<int32_t*>(topk_ids),
                    logits + kExperts, kLogitStride, static_cast<uint16_t*>(shared_logit), stream, ps.block_counts,
                    split, static_cast<const float*>(bias)));
    return run_routed(p, workspace, input, static_cast<const float*>(topk_weights),
                      static_cast<const int32_t*>(topk_ids), gate_codes, gate_meta, down_codes, down_meta,
                      shared_gate_codes, shared_gate_meta, shared_down_codes, shared_down_meta,
                      static_cast<const uint16_t*>(shared_logit), static_cast<const float*>(silu),
                      static_cast<const uint16_t*>(sigmoid), 127, nullptr, nullptr, static_cast<uint16_t*>(output),
                      static_cast<uint32_t*>(flags), T, Tcap, stream, true);
}

// ---- shared expert with the reference's fixed8 semantics --------------------------
namespace {
struct Fixed8Plan { size_t dense, gu, act, down, logit, bytes; };

Fixed8Plan fixed8_plan(int Mcap) {
    Fixed8Plan p{};
    const size_t m = size_t(Mcap);
    size_t cursor = 0;
    auto add = [&](size_t& field, size_t bytes) { field = cursor; cursor = align256(cursor + bytes); };
    const size_t dense = std::max(dense_layout(Mcap, kGateN, kHidden).workspace_bytes,
                                  dense_layout(Mcap, kDownN, kInter).workspace_bytes);
    add(p.dense, dense);
    add(p.gu, m * kGateN * 2);
    add(p.act, m * kInter * 2);
    add(p.down, m * kDownN * 2);
    add(p.logit, m * 2);
    p.bytes = cursor;
    return p;
}
}  // namespace

extern "C" hipError_t ornith_shared_fixed8_get_layout(int Mcap, size_t* workspace_bytes) {
    if (!workspace_bytes || Mcap < 0 || Mcap > kMaxTokens) return hipErrorInvalidValue;
    *workspace_bytes = fixed8_plan(Mcap).bytes;
    return hipSuccess;
}

extern "C" hipError_t ornith_shared_fixed8_launch(const void* input, const void* gate_up_codes,
                                                  const void* gate_up_meta, const void* down_codes,
                                                  const void* down_meta, const void* gate_w, const void* silu,
                                                  const void* sigmoid, void* workspace, size_t bytes, void* output,
                                                  void* flags, int M, int Mcap, hipStream_t stream) {
    if (Mcap < 0 || Mcap > kMaxTokens || M < 0 || M > Mcap) return hipErrorInvalidValue;
    const Fixed8Plan p = fixed8_plan(Mcap);
    if (bytes < p.bytes) return hipErrorInvalidValue;
    if (!M) return hipSuccess;
    const Buffer buffers[] = {{input, size_t(M) * kHidden * 2, 16, false, false},
                              {gate_up_codes, size_t(kGateN) * kHidden / 2, 16, false, false},
                              {gate_up_meta, size_t(kGateN) * (kHidden / kGroup) * 4, 4, false, false},
                              {down_codes, size_t(kDownN) * kInter / 2, 16, false, false},
                              {down_meta, size_t(kDownN) * (kInter / kGroup) * 4, 4, false, false},
                              {gate_w, size_t(kHidden) * 2, 16, false, false},
                              {silu, size_t(65536) * 4, 4, false, false},
                              {sigmoid, size_t(65536) * 2, 2, false, false},
                              {workspace, bytes, 256, true, false},
                              {output, size_t(M) * kHidden * 2, 16, true, false},
                              {flags, 4, 4, true, false}};
    if (!check_buffers(buffers)) return hipErrorInvalidValue;
    auto sticky = static_cast<uint32_t*>(flags);
    auto gu = at<uint16_t>(workspace, p.gu);
    auto act = at<uint16_t>(workspace, p.act);
    auto down = at<uint16_t>(workspace, p.down);
    auto logit = at<uint16_t>(workspace, p.logit);
    void* dws = at<void>(workspace, p.dense);
    const OrnithDenseG256Layout lg = dense_layout(Mcap, kGateN, kHidden), ld = dense_layout(Mcap, kDownN, kInter);
    TRY(dense_run(input, gate_up_codes, gate_up_meta, dws, lg, at<float>(dws, lg.projection), gu, sticky, M, kGateN,
                  kHidden, 32, stream));
    TRY(launch_fixed8_act(gu, static_cast<const uint16_t*>(input), static_cast<const uint16_t*>(gate_w),
                          static_cast<const float*>(silu), act, logit, M, stream));
    TRY(dense_run(act, down_codes, down_meta, dws, ld, at<float>(dws, ld.projection), down, sticky, M, kDownN, kInter,
                  32, stream));
    return launch_fixed8_gate(down, logit, static_cast<const uint16_t*>(sigmoid), static_cast<uint16_t*>(output), M,
                              sticky, stream);
}

// ---- the whole layer without a caller workspace --------------------------------
// Scratch of ornith_moe_layer_launch_static: the layer plan at Tcap = 32 needs
// 4,784,896 bytes; 5 MiB per GPU, held for the life of the process.  In host
// code `scratch` only names the symbol: its device address comes from
// hipGetSymbolAddress, once per device, and only that address is passed on.
namespace {
constexpr int kMaxHandoffSpins = 1 << 24;
constexpr int kStaticMaxTokens = 32;
constexpr size_t kStaticScratchBytes = size_t(5) << 20;
constexpr int kMaxDevices = 64;
}  // namespace

__device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

namespace {
std::mutex g_scratch_lock;
void* g_scratch_address[kMaxDevices];

// The device address of `scratch` on the device that runs `stream`.
hipError_t scratch_address(hipStream_t stream, void** out) {
    int device = -1;
    TRY(hipStreamGetDevice(stream, &device));
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> hold(g_scratch_lock);
    if (!g_scratch_address[device]) {
        int current = -1;
        TRY(hipGetDevice(&current));
        if (current != device) TRY(hipSetDevice(device));
        void* address = nullptr;
        const hipError_t st = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
        if (current != device) TRY(hipSetDevice(current));
        if (st != hipSuccess) return st;
        if (!address) return hipErrorInvalidSymbol;
        g_scratch_address[device] = address;
    }
    *out = g_scratch_address[device];
    return hipSuccess;
}
}  // namespace

extern "C" hipError_t ornith_moe_layer_launch_static(
    const void* input, const void* router_w, const void* bias, const void* shared_gate_w, const void* gate_codes,
    const void* gate_meta, const void* down_codes, const void* down_meta, const void* shared_gate_codes,
    const void* shared_gate_meta, const void* shared_down_codes, const void* shared_down_meta, const void* silu,
    const void* sigmoid, void* topk_weights, void* topk_ids, void* shared_logit, void* output, void* flags, int T,
    hipStream_t stream) {
    if (T < 0 || T > kStaticMaxTokens) return hipErrorInvalidValue;
    if (routed_plan(kStaticMaxTokens, true, true).l.workspace_bytes > kStaticScratchBytes) return hipErrorInvalidValue;
    if (!T) return hipSuccess;
    void* ws = nullptr;
    TRY(scratch_address(stream, &ws));
    return ornith_moe_layer_launch(input, router_w, bias, shared_gate_w, gate_codes, gate_meta, down_codes, down_meta,
                                   shared_gate_codes, shared_gate_meta, shared_down_codes, shared_down_meta, silu,
                                   sigmoid, ws, kStaticScratchBytes, topk_weights, topk_ids, shared_logit, output,
                                   flags, T, kStaticMaxTokens, stream);
}

extern "C" int ornith_mi355x_abi_version(void) { return 1; }

extern "C" int ornith_mi355x_single_token_path(int path) {
    if (path < -1 || path > 1) return -1;
    if (path == -1) return g_single_token_mode.load();
    return g_single_token_mode.exchange(path);
}

extern "C" hipError_t ornith_mi355x_silu_selfcheck(void* checked_u64, void* mismatches_u32, hipStream_t stream) {
    if (!checked_u64 || !mismatches_u32 || !aligned(checked_u64, 8) || !aligned(mismatches_u32, 4))
        return hipErrorInvalidValue;
    return launch_silu_selfcheck(static_cast<unsigned long long*>(checked_u64), static_cast<uint32_t*>(mismatches_u32),
                                 stream);
}

extern "C" int ornith_mi355x_decode_route_path(int path) {
    if (path < -1 || path > 1) return -1;
    if (path == -1) return g_route_select_mode.load();
    return g_route_select_mode.exchange(path);
}

extern "C" hipError_t ornith_mi355x_stage_trace_read(void* out_u64, size_t entries, hipStream_t stream) {
    if (!out_u64 || !aligned(out_u64, 8)) return hipErrorInvalidValue;
    return layer1_stage_trace(static_cast<uint64_t*>(out_u64), entries, stream);
}

extern "C" int ornith_mi355x_handoff_spin_limit(int spins) {
    if (spins < -1 || spins > kMaxHandoffSpins) return -1;
    if (spins == -1) return g_handoff_spins.load();
    return g_handoff_spins.exchange(spins);
}

extern "C" hipError_t ornith_mi355x_workspace_reset(void* workspace, size_t bytes, hipStream_t stream) {
    if (!workspace) {
        if (bytes != 0) return hipErrorInvalidValue;
        TRY(scratch_address(stream, &workspace));
        bytes = kStaticScratchBytes;
    }
    if (!aligned(workspace, 256) || bytes % 4) return hipErrorInvalidValue;
    return launch_fill_u32(static_cast<uint32_t*>(workspace), bytes / 4, 0u, stream);
}

// =============================================================================
// Dense
// =============================================================================
extern "C" uint32_t ornith_dense_g256_abi_version(void) { return 1; }

extern "C" hipError_t ornith_dense_g256_get_layout(int Mcap, int N, int K, int bits, OrnithDenseG256Layout* out) {
    if (!out || Mcap < 0 || Mcap > kMaxTokens || !dense_shape(N, K) || bits != 8) return hipErrorInvalidValue;
    *out = dense_layout(Mcap, N, K);
    return hipSuccess;
}

extern "C" hipError_t ornith_dense_g256_launch(const void* input, const void* codes, const void* metadata,
                                               void* workspace, size_t bytes, void* output, void* flags, int M, int Mcap,
                                               int N, int K, int bits, int transform, int geometry,
                                               hipStream_t stream) {
    OrnithDenseG256Layout l{};
    if (ornith_dense_g256_get_layout(Mcap, N, K, bits, &l) != hipSuccess || M < 0 || M > Mcap || transform != 128 ||
        geometry < 0 || geometry > 2)
        return hipErrorInvalidValue;
    if (M == 0) return hipSuccess;
    if (bytes < l.workspace_bytes) return hipErrorInvalidValue;
    const Buffer buffers[] = {{input, size_t(M) * K * 2, 16, false, false},
                              {codes, size_t(N) * K / 2, 16, false, false},
                              {metadata, size_t(N) * (K / kGroup) * 4, 4, false, false},
                              {workspace, bytes, 256, true, false},
                              {output, size_t(M) * N * 2, 16, true, false},
                              {flags, 4, 4, true, false}};
    if (!check_buffers(buffers)) return hipErrorInvalidValue;
    return dense_run(input, codes, metadata, workspace, l, at<float>(workspace, l.projection),
                     static_cast<uint16_t*>(output), static_cast<uint32_t*>(flags), M, N, K, 16, stream);
}

extern "C" hipError_t ornith_dense_g256_prepare_bf16(const void* input, const void* codes, const void* metadata,
                                                     void* transformed, void* weights, void* flags, int M, int N, int K,
                                                     hipStream_t stream) {
    if (M < 0 || M > kMaxTokens || !dense_shape(N, K)) return hipErrorInvalidValue;
    if (M == 0) return hipSuccess;
    const Buffer buffers[] = {{input, size_t(M) * K * 2, 8, false, false},
                              {codes, size_t(N) * K / 2, 4, false, false},
                              {metadata, size_t(N) * (K / kGroup) * 4, 4, false, false},
                              {transformed, size_t(M) * K * 2, 8, true, false},
                              {weights, size_t(N) * K * 2, 16, true, false},
                              {flags, 4, 4, true, false}};
    if (!check_buffers(buffers)) return hipErrorInvalidValue;
    auto sticky = static_cast<uint32_t*>(flags);
    TRY(launch_transform_bf16_fast(static_cast<const uint16_t*>(input), M, K, static_cast<uint16_t*>(transformed),
                                   sticky, stream));
    return launch_dequantize_bf16(static_cast<const uint32_t*>(codes), static_cast<const uint32_t*>(metadata), N, K, 16,
                                  static_cast<uint16_t*>(weights), sticky, stream);
}

extern "C" hipError_t ornith_dense_g256_gemm_bf16(const void* input, const void* codes, const void* metadata,
                                                  void* workspace, size_t bytes, void* output, void* flags, int M,
                                                  int N, int K, hipStream_t stream) {
    if (M < 0 || M > kMaxTokens || !dense_shape(N, K)) return hipErrorInvalidValue;
    if (M == 0) return hipSuccess;
    const size_t xt_bytes = size_t(M + 15) / 16 * 16 * K * 2;
    const Buffer buffers[] = {{input, size_t(M) * K * 2, 16, false, false},
                              {codes, size_t(N) * K / 2, 4, false, false},
                              {metadata, size_t(N) * (K / kGroup) * 4, 4, false, false},
                              {workspace, bytes, 256, true, false},
                              {output, size_t(M) * N * 2, 16, true, false},
                              {flags, 4, 4, true, false}};
    if (bytes < xt_bytes || !check_buffers(buffers)) return hipErrorInvalidValue;
    auto sticky = static_cast<uint32_t*>(flags);
    auto xt = static_cast<uint16_t*>(workspace);
    // the rest of the workspace holds the fp32 slice sums of a split K
    const size_t partial_at = align256(xt_bytes);
    float* partial = bytes > partial_at ? at<float>(workspace, partial_at) : nullptr;
    TRY(launch_transform_bf16_frag(static_cast<const uint16_t*>(input), M, K, xt, sticky, stream));
    return launch_dense_gemm_bf16(xt, static_cast<const uint32_t*>(codes), static_cast<const uint32_t*>(metadata), M, N,
                                  K, static_cast<uint16_t*>(output), partial, partial ? bytes - partial_at : 0, sticky,
                                  stream);
}

extern "C" hipError_t ornith_dense_g256_launch_n32(const void* input, const void* codes, const void* metadata,
                                                   void* workspace, size_t bytes, void* output, void* flags, int M,
                                                   int Mcap, int N, int K, int bits, int transform, int geometry,
                                                   hipStream_t stream) {
    OrnithDenseG256Layout l{};
    if (M < 1 || M > 16 || M > Mcap || N % 32 || transform != 128 || geometry != 2 ||
        ornith_dense_g256_get_layout(Mcap, N, K, bits, &l) != hipSuccess || bytes < l.workspace_bytes)
        return hipErrorInvalidValue;
    if (!input || !codes || !metadata || !workspace || !output || !flags || !aligned(input, 16) || !aligned(codes, 16) ||
        !aligned(workspace, 256))
        return hipErrorInvalidValue;
    return dense_run(input, codes, metadata, workspace, l, at<float>(workspace, l.projection),
                     static_cast<uint16_t*>(output), static_cast<uint32_t*>(flags), M, N, K, 32, stream);
}

extern "C" int ornith_dense_g256_n32_rows(void) { return 16; }

// head workspace: A8 activation words, scales, sums, then the argmax partials
// (value, index) of every row: one per 128-column block (more than 32 rows) or
// per streaming wave (at most one per 64 columns)
namespace {
constexpr int kHeadPartCols = 64;
size_t head_partials(int Mcap, int N) { return size_t(Mcap) * size_t((N + kHeadPartCols - 1) / kHeadPartCols); }
}  // namespace

extern "C" size_t ornith_dense_g256_head_workspace_bytes(int Mcap, int N) {
    if (Mcap < 0 || Mcap > 64 || N < 0) return 0;
    const size_t m = size_t(Mcap);
    return align256(m * kHidden) + align256(m * (kHidden / kGroup) * 2) + align256(m * (kHidden / kGroup) * 4) +
           2 * align256(head_partials(Mcap, N) * 4);
}

extern "C" hipError_t ornith_dense_g256_head_launch(const void* input, const void* codes, const void* metadata,
                                                    void* workspace, size_t bytes, void* logits_f32, void* logits_bf16,
                                                    void* argmax_i64, void* flags, int M, int Mcap, int N,
                                                    hipStream_t stream) {
    if (Mcap < 1 || Mcap > 64 || M < 0 || M > Mcap || N <= 0 || N % 32 || N > 262144) return hipErrorInvalidValue;
    if (bytes < ornith_dense_g256_head_workspace_bytes(Mcap, N)) return hipErrorInvalidValue;
    if (M == 0) return hipSuccess;
    if (!input || !codes || !metadata || !workspace || !logits_f32 || !argmax_i64 || !flags || !aligned(input, 16) ||
        !aligned(codes, 16) || !aligned(workspace, 256) || !aligned(logits_f32, 16) ||
        (logits_bf16 && !aligned(logits_bf16, 8)) || !aligned(argmax_i64, 8))
        return hipErrorInvalidValue;
    const size_t m = size_t(Mcap);
    const size_t scales = align256(m * kHidden), sums = scales + align256(m * (kHidden / kGroup) * 2);
    const size_t vals = sums + align256(m * (kHidden / kGroup) * 4);
    const size_t idxs = vals + align256(head_partials(Mcap, N) * 4);
    auto w = at<uint32_t>(workspace, 0);
    auto sc = at<uint16_t>(workspace, scales);
    auto su = at<int32_t>(workspace, sums);
    TRY(launch_act_bf16(static_cast<const uint16_t*>(input), kHidden, M, kHidden, 127, nullptr, w, sc, su,
                        static_cast<uint32_t*>(flags), kDenseNonfiniteInput, kDenseInvalidActivation, stream));
    MfmaArgs a{};
    a.R = M;
    a.codes = static_cast<const uint32_t*>(codes);
    a.meta = static_cast<const uint32_t*>(metadata);
    a.act_words = w; a.act_scales = sc; a.act_sums = su;
    a.K = kHidden;
    a.N = N;
    a.out = static_cast<float*>(logits_f32);
    a.out_bf16 = static_cast<uint16_t*>(logits_bf16);
    a.arg_val = at<float>(workspace, vals);
    a.arg_idx = at<int32_t>(workspace, idxs);
    a.sticky = static_cast<uint32_t*>(flags);
    a.flag_projection = kDenseNonfiniteProjection;
    a.flag_bf16 = kDenseNonfiniteBf16;
    return launch_head_mfma(a, static_cast<int64_t*>(argmax_i64), stream);
}
