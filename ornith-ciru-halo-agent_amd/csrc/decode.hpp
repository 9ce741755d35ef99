// Decode-path (T <= 32) arguments and launcher.
#pragma once
#include "kernels.hpp"
#include <atomic>

namespace ornith {

constexpr int kDecodeMaxTokens = 32;
constexpr int kLogitStride = kExperts + 1;
constexpr int64_t kGateBankWords = int64_t(2 * kInter) * kHidden / 8;
constexpr int64_t kGateBankMeta = int64_t(2 * kInter) * (kHidden / kGroup);
constexpr int64_t kDownBankWords = int64_t(kHidden) * kInter / 8;
constexpr int64_t kDownBankMeta = int64_t(kHidden) * (kInter / kGroup);

// Hand-off words of the single-token layer kernel (decode1.hip): router
// logit e at kLayer1Spread * e, middle rows of the nine slots at
// kLayer1Middle, block L's arrival word at kLayer1Arrive + kLayer1Spread * L.
// Words that different blocks write sit 64 bytes apart: 257 single-word
// stores into a few shared cache lines serialise (measured ~0.85 us more
// before the last reader sees them); each producer of the middle rows writes
// a whole 128-byte line.
constexpr int kLayer1Blocks = 256;
constexpr int kLayer1Spread = 8;
constexpr int kLayer1Middle = kLayer1Spread * 320;
constexpr int kLayer1Arrive = kLayer1Middle + (kTop + 1) * kInter;
constexpr int kLayer1Words = kLayer1Arrive + kLayer1Spread * kLayer1Blocks;
// Hand-off words of the 2..32-token route kernel (decode.hip), in the same
// region: logit (row e, token t) at kDecodeRouteLogit + 32 e + t (a router
// wave's 8 tokens are one 64-byte run), token t's expert id of slot s at
// kDecodeRouteIds + 8 t + s, block L's arrival word at kDecodeRouteArrive + 8 L.
constexpr int kDecodeRouteLogit = 0;
constexpr int kDecodeRouteIds = kDecodeRouteLogit + (kExperts + 1) * kDecodeMaxTokens;
constexpr int kDecodeRouteArrive = kDecodeRouteIds + kDecodeMaxTokens * kTop;
constexpr int kDecodeRouteMaxBlocks = 320;
constexpr int kDecodeRouteWords = kDecodeRouteArrive + 8 * kDecodeRouteMaxBlocks;
constexpr int kHandoffWords = kLayer1Words > kDecodeRouteWords ? kLayer1Words : kDecodeRouteWords;
// Stage trace of the single-token layer kernel (measurement builds only):
// kStageSlots timestamps per block for each of kStageCalls calls.
constexpr int kStageSlots = 16;
constexpr int kStageCalls = 64;
// sticky flag of this library: a block of a one-launch kernel (single-token
// layer, 2..32-token route) gave up waiting for another block's hand-off (the
// grid was not resident at once)
constexpr uint32_t kFlagHandoffTimeout = 64;

struct DecodeArgs {
    int T;
    const uint16_t* x;                 // [T, 2048] bf16
    // router (layer entry)
    const uint16_t* router_w;          // [256, 2048] bf16
    const float* bias;                 // [256] or null
    const uint16_t* shared_gate_w;     // [2048] bf16
    float* topk_w; int32_t* topk_ids;  // outputs [T, 8]
    // caller routing (routed entries)
    const int32_t* ids_in;
    // routing used by the reduce (= topk outputs or the caller's)
    const float* reduce_w; const int32_t* reduce_ids;
    // banks
    const uint32_t *w13_codes, *w13_meta, *w2_codes, *w2_meta;
    const uint32_t *s13_codes, *s13_meta, *s2_codes, *s2_meta;
    const float* silu_table; const uint16_t* sigmoid_table;
    uint16_t* shared_logit;            // bf16 [T]: written by the router, else read
    // workspace
    uint32_t* x_words; uint16_t* x_scales; int32_t* x_sums;
    float* middle;                     // [RS, 512]
    float* route_out;                  // [RS, 2048]
    float* logits; Segment* segments; int32_t* routes; int32_t* nseg;
    // one-launch kernels (single-token layer, 2..32-token route): call
    // sequence number and tagged hand-off words (kHandoffWords)
    uint32_t* l1_seq; uint64_t* l1_words;
    int handoff_spins;                 // poll rounds before a hand-off wait gives up (g_handoff_spins)
    // outputs
    float* final_f32; uint16_t* out; uint16_t* shared_out; uint16_t* layer_out;
    uint32_t* sticky;
};

size_t decode_scratch_bytes();
void carve_decode(void* base, DecodeArgs& a);
hipError_t launch_decode(const DecodeArgs& a, bool router, bool shared, int qmax, hipStream_t s);
// single-token path: 0 automatic (one launch where the grid is resident), 1 three kernels
extern std::atomic<int> g_single_token_mode;
// 2..32 tokens with the router: 0 automatic (route, top-k and sort in one launch
// where the grid is resident), 1 three kernels
extern std::atomic<int> g_route_select_mode;
hipError_t launch_decode1(const DecodeArgs& a, bool router, bool shared, int qmax, hipStream_t s);
// Copies the single-token stage trace (kStageCalls x kLayer1Blocks x
// kStageSlots words) to device memory `out`; hipErrorNotSupported unless the
// library was built with ORNITH_STAGE_TRACE.
hipError_t layer1_stage_trace(uint64_t* out, size_t entries, hipStream_t s);
// Poll rounds of the one-launch kernels' hand-off waits (default kHandoffSpins;
// 0 makes every wait give up at once, for tests of the time-out path).
extern std::atomic<int> g_handoff_spins;

}  // namespace ornith
